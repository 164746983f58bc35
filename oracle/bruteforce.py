"""Float64 brute-force oracle (numpy). TEST INFRASTRUCTURE ONLY: imported by tests/, smoke() and bench.py's CPU
baseline, never by the product.

Restates, in float64, the reference operator's arithmetic:
  corner rule       csrc/ma_deform_fused.cu:81-100 (x = loc_x * W_l - 0.5, clamp to [-2, W_l + 1], floor, 4 corners,
                    in-map test including 0 <= t < N, weight = attn * bilinear weights)
  weighted sum      csrc/ma_deform_fused.cu:228-232 (project order) and :131-146 / :170-207 (fused order)
  composition       marearts_tinydeform/reference.py:13-40 (value = memory @ W^T + b, then sample, output [B, Q, H*D])
Every function accepts numpy arrays or CPU torch tensors (converted exactly to float64).
"""

import numpy as np


def _f64(a):
    if a is None:
        return None
    if hasattr(a, 'detach'):  # torch tensor: exact conversion (half/bfloat16 values are representable in float64)
        a = a.detach().cpu().double().numpy()
    return np.asarray(a, dtype=np.float64)


def _i64(a):
    if hasattr(a, 'detach'):
        a = a.detach().cpu().numpy()
    return np.asarray(a, dtype=np.int64)


def corner_table_v2(spatial_shapes, level_start_index, sampling_locations, attention_weights, num_tokens,
                    points_per_level, method='default', padding_mask=None):
    """Corner tokens and weights for samples with per-level point counts: loc [B, Q, H, J, 2], attn [B, Q, H, J],
    J = sum(points_per_level), sample j on level level_of[j]. Returns tok, wt of shape [B, Q, H, J * 4].

    method 'default': the bilinear corner rule of corner_table. method 'discrete' (D-FINE, transformers
    models/d_fine/modeling_d_fine.py:188-206): one tap at (int(x * W + 0.5), int(y * H + 0.5)) truncated toward
    zero and clamped into the map, weight = the attention weight (a NaN coordinate takes pixel 0); the other three
    corners are empty.
    """
    shapes = _i64(spatial_shapes)
    starts = _i64(level_start_index)
    loc = _f64(sampling_locations)   # [B, Q, H, J, 2]
    attn = _f64(attention_weights)   # [B, Q, H, J]
    level_of = np.repeat(np.arange(len(points_per_level)), points_per_level)
    hl_i = shapes[level_of, 0]
    wl_i = shapes[level_of, 1]
    st = starts[level_of]
    hl, wl = hl_i.astype(np.float64), wl_i.astype(np.float64)
    B, Q, H, J = attn.shape
    if method == 'discrete':
        fx = np.fmin(np.fmax(loc[..., 0] * wl + 0.5, -1.0), wl)
        fy = np.fmin(np.fmax(loc[..., 1] * hl + 0.5, -1.0), hl)
        xi = np.clip(np.trunc(fx).astype(np.int64), 0, wl_i - 1)
        yi = np.clip(np.trunc(fy).astype(np.int64), 0, hl_i - 1)
        t = st + yi * wl_i + xi
        inside = (wl_i > 0) & (hl_i > 0) & (t >= 0) & (t < num_tokens)
        empty_t = np.full_like(t, -1)
        toks = [np.where(inside, t, -1), empty_t, empty_t, empty_t]
        zero = np.zeros_like(attn)
        wts = [np.where(inside, attn, 0.0), zero, zero, zero]
    elif method == 'default':
        x = loc[..., 0] * wl - 0.5
        y = loc[..., 1] * hl - 0.5
        # clamp before the integer conversion; np.fmax/np.fmin return the non-NaN operand, so NaN -> -2
        x = np.fmin(np.fmax(x, -2.0), wl + 1.0)
        y = np.fmin(np.fmax(y, -2.0), hl + 1.0)
        xf, yf = np.floor(x), np.floor(y)
        fx, fy = x - xf, y - yf
        x0, y0 = xf.astype(np.int64), yf.astype(np.int64)
        toks, wts = [], []
        for k in range(4):
            dx, dy = k & 1, k >> 1
            xi, yi = x0 + dx, y0 + dy
            t = st + yi * wl_i + xi
            inside = (xi >= 0) & (xi < wl_i) & (yi >= 0) & (yi < hl_i) & (t >= 0) & (t < num_tokens)
            bw = (fx if dx else 1.0 - fx) * (fy if dy else 1.0 - fy)
            toks.append(np.where(inside, t, -1))
            wts.append(np.where(inside, attn * bw, 0.0))
    else:
        raise ValueError(method)
    tok = np.stack(toks, axis=-1)  # [B, Q, H, J, 4]
    wt = np.stack(wts, axis=-1)
    if padding_mask is not None:
        pm = np.asarray(padding_mask.detach().cpu().numpy() if hasattr(padding_mask, 'detach') else padding_mask,
                        dtype=bool)
        padded = pm[np.arange(B)[:, None, None, None, None], np.maximum(tok, 0)] & (tok >= 0)
        tok = np.where(padded, -1, tok)
        wt = np.where(padded, 0.0, wt)
    return tok.reshape(B, Q, H, J * 4), wt.reshape(B, Q, H, J * 4)


def corner_table(spatial_shapes, level_start_index, sampling_locations, attention_weights, num_tokens,
                 padding_mask=None):
    """Token index and weight of every bilinear corner: tok, wt of shape [B, Q, H, L * P * 4].

    Corner order is (level, point, k) with k = dy * 2 + dx (reference csrc/ma_deform_fused.cu:93-99).
    tok is -1 and wt is 0 for corners outside the level map or outside [0, num_tokens), and for corners on tokens
    that padding_mask ([B, N], True = padded) marks.
    """
    loc = _f64(sampling_locations)   # [B, Q, H, L, P, 2]
    attn = _f64(attention_weights)   # [B, Q, H, L, P]
    B, Q, H, L, P = attn.shape
    return corner_table_v2(spatial_shapes, level_start_index, loc.reshape(B, Q, H, L * P, 2),
                           attn.reshape(B, Q, H, L * P), num_tokens, [P] * L, 'default', padding_mask)


def project(memory, value_weight, value_bias):
    """value = memory @ W^T + b in float64: [B, N, H * D]."""
    value = _f64(memory) @ _f64(value_weight).T
    if value_bias is not None:
        value = value + _f64(value_bias)
    return value


def _gather(value, heads, tok, wt, rows=None, chunk=None):
    """out[row, d] = sum_s wt[row, s] * value[b, tok[row, s], h*D + d] (tok = -1 contributes 0)."""
    B, N, HD = value.shape
    H = heads
    D = HD // H
    Q = tok.shape[1]
    S = tok.shape[-1]
    tok = tok.reshape(-1, S)
    wt = wt.reshape(-1, S)
    vh = value.reshape(B, N, H, D)
    flat = np.arange(B * Q * H) if rows is None else np.asarray(rows, dtype=np.int64)
    if chunk is None:  # bound the gathered [rows, S, D] block to ~128 MB
        chunk = max(1, (1 << 24) // max(S * D, 1))
    out = np.zeros((len(flat), D))
    for i in range(0, len(flat), chunk):
        r = flat[i:i + chunk]
        b, h = r // (Q * H), r % H
        t = tok[r]
        w = np.where(t >= 0, wt[r], 0.0)
        g = vh[b[:, None], np.maximum(t, 0), h[:, None], :]  # [R, S, D]
        out[i:i + chunk] = np.einsum('rs,rsd->rd', w, g)
    return out.reshape(B, Q, HD) if rows is None else out


def sample(value, heads, spatial_shapes, level_start_index, sampling_locations, attention_weights, rows=None,
           chunk=None, padding_mask=None):
    """out[b, q, h*D + d] = sum over in-map corners of wt * value[b, tok, h*D + d], float64: [B, Q, H * D].

    rows: optional array of flat row indices ((b * Q + q) * H + h); then only those rows are computed and the
    result is [len(rows), D].
    """
    value = _f64(value)
    tok, wt = corner_table(spatial_shapes, level_start_index, sampling_locations, attention_weights, value.shape[1],
                           padding_mask)
    return _gather(value, heads, tok, wt, rows, chunk)


def sample_v2(value, spatial_shapes, level_start_index, sampling_locations, attention_weights, points_per_level,
              method='default', padding_mask=None):
    """Per-level point counts and D-FINE's methods: value [B, N, H, D] or [B, N, H * D], loc [B, Q, H, J, 2],
    attn [B, Q, H, J] -> [B, Q, H * D], float64."""
    value = _f64(value)
    heads = sampling_locations.shape[2]
    value = value.reshape(value.shape[0], value.shape[1], -1)
    tok, wt = corner_table_v2(spatial_shapes, level_start_index, sampling_locations, attention_weights,
                              value.shape[1], points_per_level, method, padding_mask)
    return _gather(value, heads, tok, wt)


def deform_attn(memory, value_weight, value_bias, spatial_shapes, level_start_index, sampling_locations,
                attention_weights, rows=None, padding_mask=None):
    """The whole op in float64, project order (reference marearts_tinydeform/reference.py:13-40); padded tokens'
    corners are dropped (padding_mask, [B, N], True = padded)."""
    heads = sampling_locations.shape[2]
    value = project(memory, value_weight, value_bias)
    return sample(value, heads, spatial_shapes, level_start_index, sampling_locations, attention_weights, rows=rows,
                  padding_mask=padding_mask)


def deform_attn_fused_order(memory, value_weight, value_bias, spatial_shapes, level_start_index,
                            sampling_locations, attention_weights):
    """The whole op in float64, fused order: g = sum_s w_s memory[t_s]; out = W_h g + b_h * sum_s w_s.

    Restates csrc/ma_deform_fused.cu:6-14 (the linear reordering); equal to deform_attn up to float64 rounding.
    """
    mem = _f64(memory)
    W = _f64(value_weight)
    B, N, C = mem.shape
    H = sampling_locations.shape[2]
    HD = W.shape[0]
    D = HD // H
    tok, wt = corner_table(spatial_shapes, level_start_index, sampling_locations, attention_weights, N)
    Q = tok.shape[1]
    w = np.where(tok >= 0, wt, 0.0)
    b_idx = np.arange(B)[:, None, None, None]
    g = np.einsum('bqhs,bqhsc->bqhc', w, mem[b_idx, np.maximum(tok, 0)])  # [B, Q, H, C]
    Wh = W.reshape(H, D, C)
    out = np.einsum('bqhc,hdc->bqhd', g, Wh)
    if value_bias is not None:
        out = out + _f64(value_bias).reshape(H, D)[None, None] * w.sum(-1)[..., None]
    return out.reshape(B, Q, HD)
