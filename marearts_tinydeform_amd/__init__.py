"""marearts_tinydeform_amd: value projection + multi-scale deformable attention for DETR-style decoders on MI355X.

Drop-in for marearts_tinydeform (same functions, arguments, results and errors; reference
marearts_tinydeform/__init__.py:12-79). GPU tensors run hand-written HIP kernels for gfx950 through the C ABI of
libtinydeform.so; CPU tensors run the PyTorch reference path. Inference only.
"""

import functools
import math

import torch

from . import _native
from .reference import layer_locations_reference, ma_deform_attn_layer_reference, ma_deform_attn_reference

__all__ = ['ma_deform_attn', 'ma_deform_attn_reference', 'choose_mode', 'ma_deform_sample', 'ma_deform_sample_v2',
           'predict_us', 'cost_features', 'gap_features', 'ma_deform_attn_layer', 'ma_deform_attn_layer_reference', 'layer_locations_reference',
           'MSDeformAttnLayer', 'ma_deform_attn_train', 'ma_deform_sample_train']
__version__ = '0.1.1'  # the version of the reference API this package implements (marearts_tinydeform 0.1.1)

MODES = ('auto', 'fused', 'project')

# 'auto' compares predicted times of the two orders (reference marearts_tinydeform/__init__.py:21-46 uses one
# threshold on queries * levels * points * 4 / (tokens * head_dim); on MI355X the value GEMM is cheap next to
# gathering C-wide rows, so the crossover also moves with C and one threshold cannot place it). Per dtype, the fused
# kernel's time, the value GEMM's and the sampler's are each a linear function of terms that follow the kernels' own
# launch shapes (cost_features: the library's size rules, td_fused_plan / td_sample_plan / td_value_proj_plan, give
# the rows and tiles the busiest CU holds), and project mode is the GEMM plus the sampler plus a fitted gap. The
# coefficients are fitted by bench.py --fit-auto to MI355X (gfx950) measurements of the three kernels and both modes
# and checked on a grid of shapes the fit never saw (bench.py --holdout).
FUSED_LIMIT = {
    torch.float32: {'fused': (3.7445, 7.6027, 0.0, 7.5341, 8.5712, 0.0, 0.4613, 0.0809, 3.7466),
                    'gemm': (3.358, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 9.0783, 0.0612, 0.6669, 8.083),
                    'sample': (2.6256, 0.0528, 0.0, 0.0134, 0.1157),
                    'gap': (0.408, 0.0131, 0.1278, 0.0015)},
    torch.float16: {'fused': (3.5241, 8.2634, 0.0, 7.7144, 8.1228, 0.0, 0.4747, 0.1105, 1.7771),
                    'gemm': (4.2365, 0.1527, 1.1673, 0.1162, 0.0, 16.3373, 0.1835, 0.0, 0.0, 0.0, 0.0),
                    'sample': (2.8545, 0.056, 0.0, 0.0424, 0.0063),
                    'gap': (0.7467, 0.0183, 0.0619, 0.0436)},
}
FUSED_LIMIT[torch.bfloat16] = FUSED_LIMIT[torch.float16]
# The reference's table for GPUs of compute capability below 8 (marearts_tinydeform/__init__.py:30), kept so that code
# written against that module finds it. An (a, b) entry is the reference's rule: 'fused' while
# Q * L * P * 4 / (N * D) < a + b / B. No AMD GPU reports such a capability, so _limits never returns it here; a caller
# may also put (a, b) entries into FUSED_LIMIT to get the reference's rule back.
FUSED_LIMIT_SM75 = {torch.float32: (0.068, 0.0), torch.float16: (0.020, 0.0), torch.bfloat16: (0.132, 0.0)}

CUS, XCDS, L2_BYTES = 256, 8, 4 << 20  # MI355X: compute units, XCDs (each with its own L2), L2 bytes per XCD
_PLAN_DTYPE = {2: torch.float16, 4: torch.float32, 8: torch.float64}  # the size rules depend on the element size
# output tile (rows x columns) of each register- and LDS-tiled value-GEMM variant (td_gemm.hip pick_variant)
_GEMM_TILES = {2: (64, 128), 5: (64, 64), 9: (128, 128), 13: (128, 128), 23: (64, 32), 24: (32, 32), 25: (64, 64)}


def _rows_touched(N, L, B, Q, H, P):
    """Expected memory rows one XCD reads in one launch for uniformly spread locations: the kernels deal (image,
    query) rows to the XCDs in contiguous ranges, so an XCD samples ceil(B / 8) images, each level l (sizes taken to
    shrink 4x per level, as in FPN-style maps) receiving that XCD's share of the rows' 4 P corner reads."""
    if N <= 0 or L <= 0:
        return 0.0
    w = [4.0 ** -l for l in range(L)]
    imgs = max(1, -(-B // XCDS))
    reads = B * Q * H * P * 4 / XCDS / imgs
    return imgs * sum(n * -math.expm1(-reads / n) for n in (N * x / sum(w) for x in w))


def _beyond_l2(per_xcd_mb, fill_mb):
    """The share of an XCD's gathered bytes whose rows do not fit its L2."""
    return per_xcd_mb * max(0.0, 1.0 - L2_BYTES / 1e6 / fill_mb) if fill_mb > 0 else 0.0


def gap_features(B, Q, N, H, D, L, P, s):
    """Terms of what project mode costs beyond its GEMM and sampler timed apart: [1, value_mb, warm_sample_mb,
    warm_rows_mb]. value_mb: the projected values the GEMM writes and the sampler then reads. Timed alone, the sampler
    finds values that fit the XCDs' L2s (8 x 4 MB) still cached from its previous launch; after the GEMM it reads them
    from further out: warm_sample_mb, its corner reads, and warm_rows_mb, the value rows its XCDs touch, each times
    the share of the values those L2s could hold."""
    value = B * N * H * D * s
    warm = max(0.0, 1.0 - value / (XCDS * L2_BYTES))
    return [1.0, value / 1e6, B * Q * H * L * P * 4 * D * s / 1e6 * warm,
            XCDS * _rows_touched(N, L, B, Q, H, P) * H * D * s / 1e6 * warm]


def cost_features(B, Q, H, D, C, N, L, P, s, aligned=True):
    """The terms of each kernel's cost line, from the kernels' launch shapes (s: the element size in bytes):
      fused  [1, slices_mb, two_mb, tiles_mb, wide_mb, generic_mb, fill_mb, spill_mb, proj_mflop]
        *_mb      the C-wide corner rows the busiest CU gathers (its workgroups times the rows of the largest), in the
                  slot of the launch shape the fused size rule picks: balanced slices of one wavefront per row, rows
                  of two wavefronts, query tiles, rows wider than a wavefront, the generic kernel
        fill_mb   memory rows each XCD's L2 pulls in per launch (_rows_touched)
        spill_mb  gathered bytes per XCD whose rows do not fit its L2
        proj_mflop the busiest CU's projection work, its workgroups' rows (at least one 16-row MFMA tile each) x C x D
      gemm   [1, stream_mb, tiled_busy_gflop, tiled_mb, deep_rounds, deep_rounds_k, deep_mb, f32_busy_gflop, f32_mb,
              other_gflop, f32_direct_busy_gflop]
        terms of the kernel the value-projection size rule picks: the streaming kernel's bytes in whole 32-token steps
        per CU; the tiled 16-bit kernels' flops in the busiest CU's tile count (times the CU count) and their bytes;
        the deep-K direct-to-LDS kernels' tile rounds on the busiest CU, those times K / 1e3, and their bytes;
        float32 tiles (busiest CU and bytes, as for 16 bits; the 64 x 128 tiles that read A straight from memory in a
        slot of their own); the flops of the float32 and generic kernels
      sample [1, sample_mb, busy_mb, fill_mb, spill_mb]
        the D-wide corner rows the sampler reads, those of its busiest CU, value rows each XCD's L2 pulls in, and the
        gathered bytes per XCD beyond its L2"""
    S = 4 * L * P
    pdt = _PLAN_DTYPE.get(s, torch.float32)
    touched = _rows_touched(N, L, B, Q, H, P)
    per_xcd = B * Q * H * S / XCDS
    fp = _native.fused_plan(pdt, B, Q, N, C, H, D, L, P, aligned)
    fused = [1.0] + [0.0] * 8
    if fp[0] >= 0:
        lanes = fp[6] * (C * s // 16)
        cls = 4 if fp[0] == 1 else 3 if lanes > 64 else 2 if fp[4] == 0 else 1 if lanes == 128 else 0
        fused[1 + cls] = -(-fp[1] // CUS) * fp[5] * S * C * s / 1e6
        fused[6] = touched * C * s / 1e6
        fused[7] = _beyond_l2(per_xcd * C * s / 1e6, fused[6])
        fused[8] = -(-fp[1] // CUS) * max(fp[5], 16) * C * D * 2 / 1e6
    M, K, NO = B * N, C, H * D
    hm = s in (2, 4) and D * s <= 64 and D * s % 16 == 0  # td_project_forward's head-major value
    v = _native.value_proj_plan(pdt, M, K, NO, heads=H if hm else None, N=N if hm else None) if M * NO > 0 else -1
    mb, gf = M * (K + NO) * s / 1e6, 2.0 * M * K * NO / 1e9
    gemm = [1.0] + [0.0] * 10
    if v == 22:
        gemm[1] = -(-(-(-M // CUS)) // 32) * 32 * (K + NO) * s * CUS / 1e6
    elif v in (14, 18):
        mt, nt = -(-M // 256), -(-NO // 256)
        per = -(-(mt * nt) // XCDS)
        G = min((CUS // XCDS) // nt * nt, -(-per // nt) * nt)
        rounds = -(-per // G) if v == 18 and G > 0 else -(-(mt * -(-NO // 128)) // (2 * CUS))
        gemm[4], gemm[5], gemm[6] = rounds, rounds * K / 1e3, mb
    elif v in _GEMM_TILES:
        tm, tn = _GEMM_TILES[v]
        busy = -(-(-(-M // tm) * -(-NO // tn)) // CUS) * tm * tn * K * 2.0 * CUS / 1e9
        if s == 2:
            gemm[2], gemm[3] = busy, mb
        else:
            gemm[7 if v != 2 else 10], gemm[8], gemm[9] = busy, mb, gf
    elif v >= 0:
        gemm[9] = gf
    sample = [1.0, 0.0, 0.0, 0.0, 0.0]
    sp = _native.sample_plan(pdt, B, Q, N, H, D, L, P, hm) if M * NO > 0 else [-1] * 8
    if sp[0] >= 0:
        sample[1] = B * Q * H * S * D * s / 1e6
        sample[2] = -(-sp[0] // CUS) * sp[2] * S * D * s / 1e6
        sample[3] = touched * H * D * s / 1e6
        sample[4] = _beyond_l2(per_xcd * D * s / 1e6, sample[3])
    return fused, gemm, sample


# cost tables by GPU architecture (gcnArchName without feature suffixes)
ARCH_LIMITS = {'gfx950': FUSED_LIMIT}


def _arch(device_index):
    return torch.cuda.get_device_properties(device_index).gcnArchName.split(':')[0]


@functools.lru_cache(maxsize=None)
def _limits(device_index):
    """The cost table of a device: FUSED_LIMIT_SM75 below compute capability 8, as the reference chooses
    (marearts_tinydeform/__init__.py:33-36), otherwise the table of its architecture (gcnArchName), else
    FUSED_LIMIT."""
    major, _ = torch.cuda.get_device_capability(device_index)
    if major < 8:
        return FUSED_LIMIT_SM75
    try:
        return ARCH_LIMITS.get(_arch(device_index), FUSED_LIMIT)
    except (RuntimeError, AssertionError, AttributeError):  # no device properties (a CPU-only process)
        return FUSED_LIMIT


def predict_us(memory, value_weight, sampling_locations, table=None):
    """Predicted µs of mode 'fused' and 'project' for these shapes: {'fused': t, 'project': t}."""
    _, Q, H, L, P, _ = sampling_locations.shape
    return _predict(memory, value_weight, Q, H, L, P, table)


def _coef(memory, table=None):
    if table is None:
        table = _limits(memory.get_device()) if memory.is_cuda else FUSED_LIMIT
    return table.get(memory.dtype, table[torch.float16])


def _predict(memory, value_weight, Q, H, L, P, table=None):
    B, N, C = memory.shape
    HD = value_weight.shape[0]
    D = HD // max(H, 1)
    s = memory.element_size()
    coef = _coef(memory, table)
    if isinstance(coef, tuple):
        raise ValueError('a threshold table (a, b) gives a mode, not times: use choose_mode')
    aligned = (memory.data_ptr() | value_weight.data_ptr()) % 16 == 0
    ff, fg, fs = cost_features(B, Q, H, D, C, N, L, P, s, aligned)
    def dot(c, x):
        return sum(a * b for a, b in zip(c, x))
    return {'fused': dot(coef['fused'], ff),
            'project': dot(coef['gemm'], fg) + dot(coef['sample'], fs) +
                       dot(coef['gap'], gap_features(B, Q, N, H, D, L, P, s))}


def choose_mode(memory, value_weight, sampling_locations):
    """The mode 'auto' runs: 'fused' for few queries per image, 'project' (project every token first) for many."""
    _, Q, H, L, P, _ = sampling_locations.shape
    return _pick(memory, value_weight, Q, H, L, P)


def _pick(memory, value_weight, Q, H, L, P):
    coef = _coef(memory)
    if isinstance(coef, tuple):  # a reference-style threshold (a, b)
        B, N, _ = memory.shape
        D = value_weight.shape[0] // max(H, 1)
        a, b = coef
        return 'fused' if Q * L * P * 4 / max(N * D, 1) < a + b / max(B, 1) else 'project'
    t = _predict(memory, value_weight, Q, H, L, P)
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
        mode = _pick(memory, value_weight, Q, H, L, P)
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
        need_w = need[1] or (need[2] and ctx.has_bias)
        gm = gw = gb = None
        if need[0] and need_w:  # one call: at small sizes the two share a launch
            gm, gw, gb = _native.input_weight_grad(gv, weight, memory, with_bias=ctx.has_bias and need[2])
        elif need[0]:
            gm = _native.input_grad(gv, weight)
        elif need_w:
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
