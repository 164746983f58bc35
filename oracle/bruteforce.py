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


def corner_table(spatial_shapes, level_start_index, sampling_locations, attention_weights, num_tokens,
                 padding_mask=None):
    """Token index and weight of every bilinear corner: tok, wt of shape [B, Q, H, L * P * 4].

    Corner order is (level, point, k) with k = dy * 2 + dx (reference csrc/ma_deform_fused.cu:93-99).
    tok is -1 and wt is 0 for corners outside the level map or outside [0, num_tokens), and for corners on tokens
    that padding_mask ([B, N], True = padded) marks.
    """
    shapes = _i64(spatial_shapes)
    starts = _i64(level_start_index)
    loc = _f64(sampling_locations)   # [B, Q, H, L, P, 2]
    attn = _f64(attention_weights)   # [B, Q, H, L, P]
    hl = shapes[:, 0].astype(np.float64)[:, None]  # [L, 1] broadcast over P
    wl = shapes[:, 1].astype(np.float64)[:, None]
    x = loc[..., 0] * wl - 0.5
    y = loc[..., 1] * hl - 0.5
    # clamp before the integer conversion; np.fmax/np.fmin return the non-NaN operand, so NaN -> -2
    x = np.fmin(np.fmax(x, -2.0), wl + 1.0)
    y = np.fmin(np.fmax(y, -2.0), hl + 1.0)
    xf, yf = np.floor(x), np.floor(y)
    fx, fy = x - xf, y - yf
    x0, y0 = xf.astype(np.int64), yf.astype(np.int64)
    wl_i = shapes[:, 1][:, None]
    hl_i = shapes[:, 0][:, None]
    st = starts[:, None]
    toks, wts = [], []
    for k in range(4):
        dx, dy = k & 1, k >> 1
        xi, yi = x0 + dx, y0 + dy
        t = st + yi * wl_i + xi
        inside = (xi >= 0) & (xi < wl_i) & (yi >= 0) & (yi < hl_i) & (t >= 0) & (t < num_tokens)
        bw = (fx if dx else 1.0 - fx) * (fy if dy else 1.0 - fy)
        toks.append(np.where(inside, t, -1))
        wts.append(np.where(inside, attn * bw, 0.0))
    tok = np.stack(toks, axis=-1)  # [B, Q, H, L, P, 4]
    wt = np.stack(wts, axis=-1)
    B, Q, H, L, P = tok.shape[:5]
    if padding_mask is not None:
        pm = np.asarray(padding_mask.detach().cpu().numpy() if hasattr(padding_mask, 'detach') else padding_mask,
                        dtype=bool)
        padded = pm[np.arange(B)[:, None, None, None, None, None], np.maximum(tok, 0)] & (tok >= 0)
        tok = np.where(padded, -1, tok)
        wt = np.where(padded, 0.0, wt)
    return tok.reshape(B, Q, H, L * P * 4), wt.reshape(B, Q, H, L * P * 4)


def project(memory, value_weight, value_bias):
    """value = memory @ W^T + b in float64: [B, N, H * D]."""
    value = _f64(memory) @ _f64(value_weight).T
    if value_bias is not None:
        value = value + _f64(value_bias)
    return value


def sample(value, heads, spatial_shapes, level_start_index, sampling_locations, attention_weights, rows=None,
           chunk=None, padding_mask=None):
    """out[b, q, h*D + d] = sum over in-map corners of wt * value[b, tok, h*D + d], float64: [B, Q, H * D].

    rows: optional array of flat row indices ((b * Q + q) * H + h); then only those rows are computed and the
    result is [len(rows), D].
    """
    value = _f64(value)
    B, N, HD = value.shape
    H = heads
    D = HD // H
    tok, wt = corner_table(spatial_shapes, level_start_index, sampling_locations, attention_weights, N, padding_mask)
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
