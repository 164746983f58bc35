"""ctypes binding of libtinydeform.so (C ABI: include/tinydeform.h) and the tensor-level host entries.

fused_forward / sample_forward / value_proj (and the decoder-layer entries layer_*) take torch tensors on a HIP device, check them the way the reference's
host code does (csrc/ma_deform_fused.cu:236-266, 298-308, 333; same messages, RuntimeError), make them contiguous,
allocate the output with torch.empty on the caching allocator, and launch on the current stream of the tensors'
device. Nothing here computes on the CPU: without the library these functions raise.
"""

import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libtinydeform.so')

MAX_LEVEL_POINTS = 64
MAX_CHANNELS = 8192
INT32_MAX = 2 ** 31 - 1

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}

# every symbol include/tinydeform.h declares, with its ctypes signature
_i64, _vp, _int = ctypes.c_int64, ctypes.c_void_p, ctypes.c_int
SIGNATURES = {
    'td_version': (_int, []),
    'td_last_error': (ctypes.c_char_p, []),
    'td_fused_forward': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 8 + [_vp]),
    'td_sample_forward': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 7 + [_vp]),
    'td_fused_forward_masked': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 8 + [_vp]),
    'td_sample_forward_masked': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 7 + [_vp]),
    'td_sample_forward_v2': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 6 + [_vp, _int, _vp]),
    'td_value_proj': (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    'td_project_forward': (_int, [_int] + [_vp] * 8 + [_int, _vp, _vp] + [_i64] * 8 + [_vp]),
    'td_value_proj_heads': (_int, [_int, _vp, _vp, _vp, _vp] + [_i64] * 5 + [_vp]),
    'td_sample_forward_heads': (_int, [_int] + [_vp] * 6 + [_int, _vp] + [_i64] * 7 + [_vp]),
    'td_layer_prologue': (_int, [_int, _vp, _vp, _vp, _i64, _i64] + [_vp] * 7 + [_i64] * 6 + [_vp]),
    'td_layer_fused_forward': (_int, [_int, _vp, _vp, _vp, _i64, _i64] + [_vp] * 13 + [_i64] * 9 + [_vp]),
    'td_layer_sample_forward': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 7 + [_vp]),
    'td_sample_backward': (_int, [_int] + [_vp] * 11 + [_i64] * 7 + [_vp]),
    'td_input_grad': (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp]),
    'td_weight_grad_workspace': (_i64, [_int, _i64, _i64, _i64]),
    'td_input_weight_grad': (_int, [_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    'td_weight_grad': (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _i64, _vp]),
    'td_value_proj_plan': (_int, [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64]),
    'td_project_forward_noalloc': (_int, [_int] + [_vp] * 8 + [_int, _vp] + [_i64] * 8 + [_vp]),
    'td_fused_plan': (_int, [_int] + [_i64] * 8 + [_int, _vp]),
    'td_sample_plan': (_int, [_int] + [_i64] * 7 + [_int, _int, _vp]),
    'td_probe_empty': (_int, [_i64, _vp]),
    'td_probe_gather': (_int, [_vp, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    'td_probe_atomic': (_int, [_vp, _i64, _i64, _i64, _i64, _int, _vp]),
}

TD_E_WORKSPACE = -4  # td_layer_fused_forward: the problem needs loc_out / attn_out

load_error = None


def load(path=LIB_PATH):
    """Open the library and declare its signatures; returns the CDLL, or None (reason in load_error)."""
    global load_error
    if not os.path.exists(path):
        load_error = f'{path} is not built (run python -m marearts_tinydeform_amd._build)'
        return None
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:
        load_error = f'cannot load {path}: {e}'
        return None
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            load_error = f'{path} has no {name}: it predates these sources (rebuild it)'
            return None
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()


def _require():
    if lib is None:
        raise RuntimeError(f'marearts_tinydeform_amd was installed without its HIP extension: {load_error}')
    return lib


def _check(rc):
    if rc != 0:
        raise RuntimeError(lib.td_last_error().decode(errors='replace') or f'tinydeform error {rc}')


def _ptr(t):
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, '_cuda_getCurrentRawStream', None)


def _stream(device):
    """Handle of the current stream of `device` (torch's raw getter: ~0.1 us instead of ~2 us for a Stream)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def check_geometry(ref, spatial_shapes, level_start_index, sampling_locations, attention_weights, require_gpu=True):
    """Shape, dtype and device checks shared by both modes; returns B, Q, H, L, P.

    Same conditions and messages as the reference's check_geometry (csrc/ma_deform_fused.cu:236-266).
    require_gpu=False skips the device-type check only (the rules can then be exercised on CPU tensors).
    """
    if require_gpu and not ref.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if ref.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    if ref.size(1) > INT32_MAX:
        raise RuntimeError('too many memory tokens')
    if sampling_locations.dim() != 6 or sampling_locations.size(5) != 2:
        raise RuntimeError('sampling_locations must be [B, Q, H, L, P, 2]')
    if attention_weights.dim() != 5:
        raise RuntimeError('attention_weights must be [B, Q, H, L, P]')
    if attention_weights.shape != sampling_locations.shape[:5]:
        raise RuntimeError('attention_weights must be [B, Q, H, L, P] like sampling_locations')
    B, Q, H, L, P = sampling_locations.shape[:5]
    if ref.size(0) != B:
        raise RuntimeError('batch size mismatch')
    if H <= 0:
        raise RuntimeError('need at least one head')
    if L * P > MAX_LEVEL_POINTS:
        raise RuntimeError(f'levels x points must be <= {MAX_LEVEL_POINTS}')
    if spatial_shapes.dtype != torch.int64 or spatial_shapes.dim() != 2 or spatial_shapes.shape != (L, 2):
        raise RuntimeError('spatial_shapes must be int64 [L, 2]')
    if level_start_index.dtype != torch.int64 or level_start_index.dim() != 1 or level_start_index.size(0) != L:
        raise RuntimeError('level_start_index must be int64 [L]')
    for t in (sampling_locations, attention_weights, spatial_shapes, level_start_index):
        if t.device != ref.device:
            raise RuntimeError('all tensors must be on the same device')
    for t in (sampling_locations, attention_weights):
        if t.dtype != ref.dtype:
            raise RuntimeError('all float tensors must have the same dtype')
    if ref.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {ref.dtype}')
    if B * Q * H > INT32_MAX:
        raise RuntimeError('too many (batch, query, head) rows')
    return B, Q, H, L, P


def check_projection(memory, weight, bias, H=None):
    """value_weight / value_bias checks (reference csrc/ma_deform_fused.cu:298-308); returns HD."""
    C = memory.size(2)
    if weight.dim() != 2 or weight.size(1) != C:
        raise RuntimeError('value_weight must be [H * D, C] with C = memory.size(2)')
    HD = weight.size(0)
    if H is not None and HD % H != 0:
        raise RuntimeError('value_weight rows must be a multiple of the head count')
    if weight.device != memory.device or weight.dtype != memory.dtype:
        raise RuntimeError('value_weight must have the device and dtype of memory')
    if bias is not None and (bias.device != memory.device or bias.dtype != memory.dtype or bias.dim() != 1
                             or bias.size(0) != HD):
        raise RuntimeError('value_bias must be [H * D] like value_weight, same device and dtype')
    return HD


def check_padding_mask(ref, padding_mask):
    """padding_mask: None or bool/uint8 [B, N] on the device of ref (non-zero = padded token); returns it contiguous
    as uint8 bytes, or None."""
    if padding_mask is None:
        return None
    if padding_mask.dtype not in (torch.bool, torch.uint8) or padding_mask.shape != ref.shape[:2]:
        raise RuntimeError('padding_mask must be bool [B, N] like memory / value')
    if padding_mask.device != ref.device:
        raise RuntimeError('all tensors must be on the same device')
    return padding_mask.contiguous()


def fused_forward(memory, weight, bias, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                  padding_mask=None):
    """Fused mode (replaces the reference's _C.fused_forward, csrc/ma_deform_fused.cu:291-325)."""
    lib_ = _require()
    B, Q, H, L, P = check_geometry(memory, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    N, C = memory.size(1), memory.size(2)
    HD = check_projection(memory, weight, bias, H)
    mask = check_padding_mask(memory, padding_mask)
    if C > MAX_CHANNELS:
        raise RuntimeError(f'channels must be <= {MAX_CHANNELS}')
    dev = memory.device
    mem, w = memory.contiguous(), weight.contiguous()
    b = None if bias is None else bias.contiguous()
    lc, aw = sampling_locations.contiguous(), attention_weights.contiguous()
    sh, st = spatial_shapes.contiguous(), level_start_index.contiguous()
    out = torch.empty((B, Q, HD), dtype=memory.dtype, device=dev)
    if out.numel() == 0:
        return out
    _check(lib_.td_fused_forward_masked(DTYPE_CODES[memory.dtype], mem.data_ptr(), w.data_ptr(), _ptr(b),
                                        sh.data_ptr(), st.data_ptr(), lc.data_ptr(), aw.data_ptr(), _ptr(mask),
                                        out.data_ptr(), B, Q, N, C, H, HD // H, L, P, _stream(dev)))
    return out


def sample_forward(value, heads, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                   padding_mask=None):
    """Sampling of projected values (replaces the reference's _C.sample_forward, csrc/ma_deform_fused.cu:327-350)."""
    lib_ = _require()
    B, Q, H, L, P = check_geometry(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    N, HD = value.size(1), value.size(2)
    if heads != H or HD % H != 0:
        raise RuntimeError('value must be [B, N, H * D] with H = sampling_locations.size(2)')
    mask = check_padding_mask(value, padding_mask)
    dev = value.device
    v = value.contiguous()
    lc, aw = sampling_locations.contiguous(), attention_weights.contiguous()
    sh, st = spatial_shapes.contiguous(), level_start_index.contiguous()
    out = torch.empty((B, Q, HD), dtype=value.dtype, device=dev)
    if out.numel() == 0:
        return out
    _check(lib_.td_sample_forward_masked(DTYPE_CODES[value.dtype], v.data_ptr(), sh.data_ptr(), st.data_ptr(),
                                         lc.data_ptr(), aw.data_ptr(), _ptr(mask), out.data_ptr(), B, Q, N, H, HD // H,
                                         L, P, _stream(dev)))
    return out


def sample_forward_v2(value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                      num_points_list, method='default', padding_mask=None):
    """Sampling with per-level point counts and D-FINE's methods (td_sample_forward_v2)."""
    lib_ = _require()
    if method not in ('default', 'discrete'):
        raise ValueError(f"method must be 'default' or 'discrete', got {method!r}")
    if not value.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if value.dim() == 4:
        value = value.flatten(2)
    if value.dim() != 3:
        raise RuntimeError('value must be [B, N, H * D] or [B, N, H, D]')
    if sampling_locations.dim() != 5 or sampling_locations.size(4) != 2:
        raise RuntimeError('sampling_locations must be [B, Q, H, sum(num_points_list), 2]')
    B, Q, H, J = sampling_locations.shape[:4]
    points = [int(n) for n in num_points_list]
    L = len(points)
    if sum(points) != J or any(n < 0 for n in points):
        raise RuntimeError('sampling_locations must have sum(num_points_list) samples per head')
    if J > MAX_LEVEL_POINTS:
        raise RuntimeError(f'levels x points must be <= {MAX_LEVEL_POINTS}')
    if attention_weights.shape != sampling_locations.shape[:4]:
        raise RuntimeError('attention_weights must be [B, Q, H, sum(num_points_list)] like sampling_locations')
    if value.size(0) != B:
        raise RuntimeError('batch size mismatch')
    N, HD = value.size(1), value.size(2)
    if H <= 0 or HD % H != 0:
        raise RuntimeError('value must be [B, N, H * D] with H = sampling_locations.size(2)')
    if spatial_shapes.dtype != torch.int64 or spatial_shapes.shape != (L, 2):
        raise RuntimeError('spatial_shapes must be int64 [L, 2]')
    if level_start_index.dtype != torch.int64 or level_start_index.shape != (L,):
        raise RuntimeError('level_start_index must be int64 [L]')
    for t in (sampling_locations, attention_weights, spatial_shapes, level_start_index):
        if t.device != value.device:
            raise RuntimeError('all tensors must be on the same device')
    for t in (sampling_locations, attention_weights):
        if t.dtype != value.dtype:
            raise RuntimeError('all float tensors must have the same dtype')
    if value.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {value.dtype}')
    mask = check_padding_mask(value, padding_mask)
    dev = value.device
    v = value.contiguous()
    lc, aw = sampling_locations.contiguous(), attention_weights.contiguous()
    sh, st = spatial_shapes.contiguous(), level_start_index.contiguous()
    out = torch.empty((B, Q, HD), dtype=value.dtype, device=dev)
    if out.numel() == 0:
        return out
    pts = (ctypes.c_int64 * max(L, 1))(*points)
    _check(lib_.td_sample_forward_v2(DTYPE_CODES[value.dtype], v.data_ptr(), sh.data_ptr(), st.data_ptr(),
                                     lc.data_ptr(), aw.data_ptr(), _ptr(mask), out.data_ptr(), B, Q, N, H, HD // H, L,
                                     ctypes.cast(pts, ctypes.c_void_p), int(method == 'discrete'), _stream(dev)))
    return out


def value_proj(memory, weight, bias):
    """value = memory @ weight^T + bias on the library's GEMM (replaces F.linear, marearts_tinydeform/__init__.py:77)."""
    lib_ = _require()
    if not memory.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if memory.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    if memory.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {memory.dtype}')
    HD = check_projection(memory, weight, bias)
    B, N, C = memory.shape
    dev = memory.device
    mem, w = memory.contiguous(), weight.contiguous()
    b = None if bias is None else bias.contiguous()
    value = torch.empty((B, N, HD), dtype=memory.dtype, device=dev)
    if value.numel() == 0:
        return value
    _check(lib_.td_value_proj(DTYPE_CODES[memory.dtype], mem.data_ptr(), w.data_ptr(), _ptr(b), value.data_ptr(),
                              B * N, C, HD, _stream(dev)))
    return value


def value_proj_plan(dtype, M, K, NO, bias=True, offsets=None, heads=None, N=None):
    """The tile variant td_value_proj (or, with heads and N, td_value_proj_heads) launches for an [M, K] x [NO, K]^T
    problem (0: the generic VALU kernel). offsets: byte offsets from a 256-byte boundary of the memory, weight, bias
    and value pointers, as a dict with any of those keys (default 0); bias=False: no bias. No memory is touched."""
    lib_ = _require()
    off = {'memory': 0, 'weight': 0, 'bias': 0, 'value': 0}
    off.update(offsets or {})
    base = 1 << 20
    ptrs = [base * (i + 1) + off[k] for i, k in enumerate(('memory', 'weight', 'bias', 'value'))]
    if not bias:
        ptrs[2] = None
    rc = lib_.td_value_proj_plan(DTYPE_CODES[dtype], *ptrs, M, K, NO, N or 0, heads or 0)
    if rc < 0:
        _check(rc)
    return rc


def _check_locations(ref, spatial_shapes, level_start_index, loc, attn, loc_acc):
    """Geometry checks for the project-mode entries; returns B, Q, H, L, P. loc_acc=False: loc / attn in ref's dtype,
    checked as the reference does (csrc/ma_deform_fused.cu:236-266); True: in float32 (float64 for float64), as
    layer_prologue writes them."""
    if not loc_acc:
        return check_geometry(ref, spatial_shapes, level_start_index, loc, attn)
    if not ref.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if loc.dim() != 6 or loc.size(5) != 2 or attn.shape != loc.shape[:5]:
        raise RuntimeError('sampling_locations must be [B, Q, H, L, P, 2]')
    B, Q, H, L, P = loc.shape[:5]
    acc = acc_dtype(ref.dtype)
    if loc.dtype != acc or attn.dtype != acc:
        raise RuntimeError(f'locations and weights must be {acc} for {ref.dtype} values')
    if ref.size(0) != B:
        raise RuntimeError('batch size mismatch')
    if spatial_shapes.dtype != torch.int64 or spatial_shapes.shape != (L, 2):
        raise RuntimeError('spatial_shapes must be int64 [L, 2]')
    if level_start_index.dtype != torch.int64 or level_start_index.shape != (L,):
        raise RuntimeError('level_start_index must be int64 [L]')
    for t in (loc, attn, spatial_shapes, level_start_index):
        if t.device != ref.device:
            raise RuntimeError('all tensors must be on the same device')
    if ref.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {ref.dtype}')
    return B, Q, H, L, P


def project_forward(memory, weight, bias, spatial_shapes, level_start_index, loc, attn, padding_mask=None,
                    loc_acc=False):
    """Project mode in one call (td_project_forward): value projection into a scratch buffer, then sampling.
    loc_acc as in _check_locations."""
    lib_ = _require()
    if memory.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    B, Q, H, L, P = _check_locations(memory, spatial_shapes, level_start_index, loc, attn, loc_acc)
    HD = check_projection(memory, weight, bias, H)
    mask = check_padding_mask(memory, padding_mask)
    N, C = memory.size(1), memory.size(2)
    dev = memory.device
    mem, w, b, lc, aw, sh, st = _contig(memory, weight, bias, loc, attn, spatial_shapes, level_start_index)
    out = torch.empty((B, Q, HD), dtype=memory.dtype, device=dev)
    if out.numel() == 0:
        return out
    ws = torch.empty((B * N * HD,), dtype=memory.dtype, device=dev)
    _check(lib_.td_project_forward(DTYPE_CODES[memory.dtype], mem.data_ptr(), w.data_ptr(), _ptr(b), sh.data_ptr(),
                                   st.data_ptr(), lc.data_ptr(), aw.data_ptr(), _ptr(mask), 1 if loc_acc else 0,
                                   ws.data_ptr(), out.data_ptr(), B, Q, N, C, H, HD // H, L, P, _stream(dev)))
    return out


NOALLOC_SCRATCH_BYTES = 64 << 20  # TD_NOALLOC_SCRATCH_BYTES


def project_forward_noalloc(memory, weight, bias, spatial_shapes, level_start_index, loc, attn, padding_mask=None,
                            loc_acc=False, out=None):
    """Project mode without a workspace (td_project_forward_noalloc): the projected values go to the library's
    static per-GPU scratch array (NOALLOC_SCRATCH_BYTES), so the library allocates nothing; out (optional) is the
    caller's [B, Q, H*D] output. Calls that overlap on one GPU race on the scratch array."""
    lib_ = _require()
    if memory.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    B, Q, H, L, P = _check_locations(memory, spatial_shapes, level_start_index, loc, attn, loc_acc)
    HD = check_projection(memory, weight, bias, H)
    mask = check_padding_mask(memory, padding_mask)
    N, C = memory.size(1), memory.size(2)
    dev = memory.device
    mem, w, b, lc, aw, sh, st = _contig(memory, weight, bias, loc, attn, spatial_shapes, level_start_index)
    if out is None:
        out = torch.empty((B, Q, HD), dtype=memory.dtype, device=dev)
    elif out.shape != (B, Q, HD) or out.dtype != memory.dtype or out.device != dev or not out.is_contiguous():
        raise RuntimeError('out must be a contiguous [B, Q, H*D] tensor of the memory dtype on its device')
    if out.numel() == 0:
        return out
    with torch.cuda.device(dev):  # the library resolves its scratch array on the current device
        _check(lib_.td_project_forward_noalloc(DTYPE_CODES[memory.dtype], mem.data_ptr(), w.data_ptr(), _ptr(b),
                                               sh.data_ptr(), st.data_ptr(), lc.data_ptr(), aw.data_ptr(), _ptr(mask),
                                               1 if loc_acc else 0, out.data_ptr(), B, Q, N, C, H, HD // H, L, P,
                                               _stream(dev)))
    return out


def value_proj_heads(memory, weight, bias, heads):
    """Head-major value projection (td_value_proj_heads): [B, N, C] -> [B, H, N, D]."""
    lib_ = _require()
    if not memory.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if memory.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    if memory.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {memory.dtype}')
    HD = check_projection(memory, weight, bias, heads)
    B, N, C = memory.shape
    D = HD // heads
    if D * memory.element_size() % 16 != 0:
        raise RuntimeError('head-major values need a head row of a multiple of 16 bytes')
    mem, w, b = _contig(memory, weight, bias)
    value = torch.empty((B, heads, N, D), dtype=memory.dtype, device=memory.device)
    if value.numel() == 0:
        return value
    _check(lib_.td_value_proj_heads(DTYPE_CODES[memory.dtype], mem.data_ptr(), w.data_ptr(), _ptr(b),
                                    value.data_ptr(), B, N, C, heads, D, _stream(memory.device)))
    return value


def sample_forward_heads(value, spatial_shapes, level_start_index, loc, attn, padding_mask=None, loc_acc=False):
    """Sampling of a head-major value [B, H, N, D] (td_sample_forward_heads) -> [B, Q, H * D]."""
    lib_ = _require()
    if value.dim() != 4:
        raise RuntimeError('value must be [B, H, N, D]')
    B_, H_, N, D = value.shape
    flat = value.view(B_, N, H_ * D) if value.is_contiguous() else value.reshape(B_, N, H_ * D)
    B, Q, H, L, P = _check_locations(flat, spatial_shapes, level_start_index, loc, attn, loc_acc)
    if H != H_:
        raise RuntimeError('value must be [B, H, N, D] with H = sampling_locations.size(2)')
    mask = check_padding_mask(flat, padding_mask)
    v, lc, aw, sh, st = _contig(value, loc, attn, spatial_shapes, level_start_index)
    out = torch.empty((B, Q, H * D), dtype=value.dtype, device=value.device)
    if out.numel() == 0:
        return out
    _check(lib_.td_sample_forward_heads(DTYPE_CODES[value.dtype], v.data_ptr(), sh.data_ptr(), st.data_ptr(),
                                        lc.data_ptr(), aw.data_ptr(), _ptr(mask), 1 if loc_acc else 0,
                                        out.data_ptr(), B, Q, N, H, D, L, P, _stream(value.device)))
    return out


def sample_backward(value, heads, spatial_shapes, level_start_index, sampling_locations, attention_weights, grad_out,
                    padding_mask=None):
    """Gradients of sample_forward (td_sample_backward): (grad_value [B, N, H * D], grad_loc, grad_attn), each in the
    input dtype; grad_value is accumulated in float32 (float64) and rounded once."""
    lib_ = _require()
    B, Q, H, L, P = check_geometry(value, spatial_shapes, level_start_index, sampling_locations, attention_weights)
    N, HD = value.size(1), value.size(2)
    if heads != H or HD % H != 0:
        raise RuntimeError('value must be [B, N, H * D] with H = sampling_locations.size(2)')
    if HD // H > 256:
        raise RuntimeError('sample backward: head dim must be <= 256')
    if grad_out.shape != (B, Q, HD) or grad_out.dtype != value.dtype or grad_out.device != value.device:
        raise RuntimeError('grad_out must be [B, Q, H * D] like the forward output')
    mask = check_padding_mask(value, padding_mask)
    dev, dt = value.device, value.dtype
    v, go = value.contiguous(), grad_out.contiguous()
    lc, aw = sampling_locations.contiguous(), attention_weights.contiguous()
    sh, st = spatial_shapes.contiguous(), level_start_index.contiguous()
    acc = torch.empty((B, N, HD), dtype=acc_dtype(dt), device=dev)
    gv = acc if acc.dtype == dt else torch.empty((B, N, HD), dtype=dt, device=dev)
    gl = torch.empty_like(lc)
    ga = torch.empty_like(aw)
    if acc.numel() == 0 and gl.numel() == 0:
        return gv, gl, ga
    _check(lib_.td_sample_backward(DTYPE_CODES[dt], v.data_ptr(), sh.data_ptr(), st.data_ptr(), lc.data_ptr(),
                                   aw.data_ptr(), _ptr(mask), go.data_ptr(), acc.data_ptr(), gv.data_ptr(),
                                   gl.data_ptr(), ga.data_ptr(), B, Q, N, H, HD // H, L, P, _stream(dev)))
    return gv, gl, ga


def input_grad(grad_value, weight):
    """grad_memory = grad_value @ weight on the library's GEMM (td_input_grad): [B, N, C]."""
    lib_ = _require()
    B, N, HD = grad_value.shape
    C = weight.size(1)
    if weight.shape != (HD, C) or weight.dtype != grad_value.dtype or weight.device != grad_value.device:
        raise RuntimeError('weight must be [H * D, C] like value_weight')
    dev = grad_value.device
    g, w = grad_value.contiguous(), weight.contiguous()
    wt = torch.empty((C, HD), dtype=w.dtype, device=dev)
    out = torch.empty((B, N, C), dtype=g.dtype, device=dev)
    if out.numel() == 0:
        return out
    if HD == 0:
        return out.zero_()
    _check(lib_.td_input_grad(DTYPE_CODES[g.dtype], g.data_ptr(), w.data_ptr(), wt.data_ptr(), out.data_ptr(), B * N,
                              HD, C, _stream(dev)))
    return out


def weight_grad(grad_value, memory, with_bias=True):
    """(grad_weight [H * D, C] = grad_value^T @ memory, grad_bias [H * D] or None) over all B * N tokens
    (td_weight_grad), with its float32 (float64) split-K workspace from the caching allocator."""
    lib_ = _require()
    B, N, HD = grad_value.shape
    C = memory.size(2)
    if memory.shape[:2] != (B, N) or memory.dtype != grad_value.dtype or memory.device != grad_value.device:
        raise RuntimeError('memory must be [B, N, C] with the tokens of grad_value')
    dev, dt = grad_value.device, grad_value.dtype
    g, mem = grad_value.contiguous(), memory.contiguous()
    gw = torch.empty((HD, C), dtype=dt, device=dev)
    gb = torch.empty((HD,), dtype=dt, device=dev) if with_bias else None
    code = DTYPE_CODES[dt]
    ws_bytes = int(lib_.td_weight_grad_workspace(code, B * N, HD, C))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    _check(lib_.td_weight_grad(code, g.data_ptr(), mem.data_ptr(), gw.data_ptr(), _ptr(gb), B * N, HD, C,
                               ws.data_ptr(), ws_bytes, _stream(dev)))
    return gw, gb


def input_weight_grad(grad_value, weight, memory, with_bias=True):
    """input_grad and weight_grad of the same grad_value in one call (td_input_weight_grad): (grad_memory [B, N, C],
    grad_weight [H * D, C], grad_bias [H * D] or None)."""
    lib_ = _require()
    B, N, HD = grad_value.shape
    C = memory.size(2)
    if weight.shape != (HD, C) or weight.dtype != grad_value.dtype or weight.device != grad_value.device:
        raise RuntimeError('weight must be [H * D, C] like value_weight')
    if memory.shape[:2] != (B, N) or memory.dtype != grad_value.dtype or memory.device != grad_value.device:
        raise RuntimeError('memory must be [B, N, C] with the tokens of grad_value')
    dev, dt = grad_value.device, grad_value.dtype
    g, w, mem = grad_value.contiguous(), weight.contiguous(), memory.contiguous()
    wt = torch.empty((C, HD), dtype=dt, device=dev)
    gm = torch.empty((B, N, C), dtype=dt, device=dev)
    gw = torch.empty((HD, C), dtype=dt, device=dev)
    gb = torch.empty((HD,), dtype=dt, device=dev) if with_bias else None
    code = DTYPE_CODES[dt]
    ws_bytes = int(lib_.td_weight_grad_workspace(code, B * N, HD, C))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    _check(lib_.td_input_weight_grad(code, g.data_ptr(), w.data_ptr(), wt.data_ptr(), mem.data_ptr(), gm.data_ptr(),
                                     gw.data_ptr(), _ptr(gb), B * N, HD, C, ws.data_ptr(), ws_bytes, _stream(dev)))
    return gm, gw, gb


def acc_dtype(dtype):
    """Type the layer entries compute locations and attention weights in: float32, or float64 for float64."""
    return torch.float64 if dtype == torch.float64 else torch.float32


def check_layer(memory, query, reference_points, offsets_weight, offsets_bias, attn_weight, attn_bias, position,
                spatial_shapes, num_heads, num_points, require_gpu=True):
    """Query-side checks of the decoder-layer entries; returns B, Q, Cq, H, L, P.

    query [B, Q, Cq] (and position, same shape, or None), reference_points [B, Q, 1 or L, 2 or 4],
    offsets_weight [H * L * P * 2, Cq] / offsets_bias [H * L * P * 2] or None, attn_weight [H * L * P, Cq] /
    attn_bias [H * L * P] or None, all on memory's device and in its dtype; L = spatial_shapes.size(0).
    """
    if require_gpu and not memory.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if memory.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    if query.dim() != 3:
        raise RuntimeError('hidden_states must be [B, Q, C]')
    B, Q, Cq = query.shape
    if memory.size(0) != B:
        raise RuntimeError('batch size mismatch')
    H, P = int(num_heads), int(num_points)
    if H <= 0:
        raise RuntimeError('need at least one head')
    if P < 0:
        raise RuntimeError('num_points must be non-negative')
    if spatial_shapes.dtype != torch.int64 or spatial_shapes.dim() != 2 or spatial_shapes.size(1) != 2:
        raise RuntimeError('spatial_shapes must be int64 [L, 2]')
    L = spatial_shapes.size(0)
    if L * P > MAX_LEVEL_POINTS:
        raise RuntimeError(f'levels x points must be <= {MAX_LEVEL_POINTS}')
    if Cq > MAX_CHANNELS:
        raise RuntimeError(f'query channels must be <= {MAX_CHANNELS}')
    if (reference_points.dim() != 4 or reference_points.shape[:2] != (B, Q) or reference_points.size(2) not in (1, L)
            or reference_points.size(3) not in (2, 4)):
        raise RuntimeError('reference_points must be [B, Q, 1 or L, 2 or 4]')
    if offsets_weight.shape != (H * L * P * 2, Cq):
        raise RuntimeError('sampling_offsets weight must be [H * L * P * 2, C]')
    if attn_weight.shape != (H * L * P, Cq):
        raise RuntimeError('attention_weights weight must be [H * L * P, C]')
    if offsets_bias is not None and offsets_bias.shape != (H * L * P * 2,):
        raise RuntimeError('sampling_offsets bias must be [H * L * P * 2]')
    if attn_bias is not None and attn_bias.shape != (H * L * P,):
        raise RuntimeError('attention_weights bias must be [H * L * P]')
    if position is not None and position.shape != query.shape:
        raise RuntimeError('position_embeddings must be [B, Q, C] like hidden_states')
    for t in (query, reference_points, offsets_weight, offsets_bias, attn_weight, attn_bias, position):
        if t is None:
            continue
        if t.device != memory.device:
            raise RuntimeError('all tensors must be on the same device')
        if t.dtype != memory.dtype:
            raise RuntimeError('all float tensors must have the same dtype')
    if spatial_shapes.device != memory.device:
        raise RuntimeError('all tensors must be on the same device')
    if memory.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {memory.dtype}')
    if B * Q * H > INT32_MAX:
        raise RuntimeError('too many (batch, query, head) rows')
    return B, Q, Cq, H, L, P


def _contig(*ts):
    return [None if t is None else t.contiguous() for t in ts]


def layer_prologue(query, position, reference_points, offsets_weight, offsets_bias, attn_weight, attn_bias,
                   spatial_shapes, num_heads, num_points):
    """Query prologue alone (td_layer_prologue): sampling locations [B, Q, H, L, P, 2] and attention weights
    [B, Q, H, L, P] in float32 (float64 for float64 inputs)."""
    lib_ = _require()
    B, Q, Cq, H, L, P = check_layer(query, query, reference_points, offsets_weight, offsets_bias, attn_weight,
                                    attn_bias, position, spatial_shapes, num_heads, num_points)
    dev = query.device
    acc = acc_dtype(query.dtype)
    loc = torch.empty((B, Q, H, L, P, 2), dtype=acc, device=dev)
    attn = torch.empty((B, Q, H, L, P), dtype=acc, device=dev)
    if attn.numel() == 0:
        return loc, attn
    q, pos, ref, ow, ob, aw, ab, sh = _contig(query, position, reference_points, offsets_weight, offsets_bias,
                                              attn_weight, attn_bias, spatial_shapes)
    _check(lib_.td_layer_prologue(DTYPE_CODES[query.dtype], q.data_ptr(), _ptr(pos), ref.data_ptr(), ref.size(2),
                                  ref.size(3), ow.data_ptr(), _ptr(ob), aw.data_ptr(), _ptr(ab), sh.data_ptr(),
                                  loc.data_ptr(), attn.data_ptr(), B, Q, Cq, H, L, P, _stream(dev)))
    return loc, attn


def layer_fused_forward(query, position, reference_points, offsets_weight, offsets_bias, attn_weight, attn_bias,
                        memory, value_weight, value_bias, spatial_shapes, level_start_index, num_heads, num_points,
                        padding_mask=None, return_locations=False):
    """Fused decoder layer core (td_layer_fused_forward): the query prologue inside the fused kernel.

    Returns out [B, Q, H * D] and, with return_locations, (loc, attn) in float32 (float64 for float64 inputs),
    else None. Problems the in-kernel prologue cannot take get location buffers and a second call."""
    lib_ = _require()
    B, Q, Cq, H, L, P = check_layer(memory, query, reference_points, offsets_weight, offsets_bias, attn_weight,
                                    attn_bias, position, spatial_shapes, num_heads, num_points)
    N, C = memory.size(1), memory.size(2)
    HD = check_projection(memory, value_weight, value_bias, H)
    if C > MAX_CHANNELS:
        raise RuntimeError(f'channels must be <= {MAX_CHANNELS}')
    if level_start_index.dtype != torch.int64 or level_start_index.shape != (L,):
        raise RuntimeError('level_start_index must be int64 [L]')
    if level_start_index.device != memory.device:
        raise RuntimeError('all tensors must be on the same device')
    mask = check_padding_mask(memory, padding_mask)
    dev = memory.device
    acc = acc_dtype(memory.dtype)
    out = torch.empty((B, Q, HD), dtype=memory.dtype, device=dev)
    loc = attn = None
    if return_locations:
        loc = torch.empty((B, Q, H, L, P, 2), dtype=acc, device=dev)
        attn = torch.empty((B, Q, H, L, P), dtype=acc, device=dev)
    if B * Q * H == 0:
        return out, ((loc, attn) if return_locations else None)
    q, pos, ref, ow, ob, aw, ab = _contig(query, position, reference_points, offsets_weight, offsets_bias, attn_weight,
                                          attn_bias)
    mem, w, b, sh, st = _contig(memory, value_weight, value_bias, spatial_shapes, level_start_index)

    def call(lo, at):
        return lib_.td_layer_fused_forward(DTYPE_CODES[memory.dtype], q.data_ptr(), _ptr(pos), ref.data_ptr(),
                                           ref.size(2), ref.size(3), ow.data_ptr(), _ptr(ob), aw.data_ptr(), _ptr(ab),
                                           mem.data_ptr(), w.data_ptr(), _ptr(b), sh.data_ptr(), st.data_ptr(),
                                           _ptr(mask), out.data_ptr(), _ptr(lo), _ptr(at), B, Q, N, Cq, C, H, HD // H,
                                           L, P, _stream(dev))

    rc = call(loc, attn)
    if rc == TD_E_WORKSPACE and loc is None:
        loc = torch.empty((B, Q, H, L, P, 2), dtype=acc, device=dev)
        attn = torch.empty((B, Q, H, L, P), dtype=acc, device=dev)
        rc = call(loc, attn)
    _check(rc)
    return out, ((loc, attn) if return_locations else None)


def layer_sample_forward(value, heads, spatial_shapes, level_start_index, loc, attn, padding_mask=None):
    """Sampling of projected values with float32 (float64) locations and weights (td_layer_sample_forward)."""
    lib_ = _require()
    if not value.is_cuda:
        raise RuntimeError('inputs must be GPU tensors')
    if value.dim() != 3:
        raise RuntimeError('memory / value must be [B, N, C]')
    if loc.dim() != 6 or loc.size(5) != 2 or attn.shape != loc.shape[:5]:
        raise RuntimeError('sampling_locations must be [B, Q, H, L, P, 2]')
    B, Q, H, L, P = loc.shape[:5]
    N, HD = value.size(1), value.size(2)
    if heads != H or HD % H != 0 or value.size(0) != B:
        raise RuntimeError('value must be [B, N, H * D] with H = sampling_locations.size(2)')
    acc = acc_dtype(value.dtype)
    if loc.dtype != acc or attn.dtype != acc:
        raise RuntimeError(f'locations and weights must be {acc} for {value.dtype} values')
    if spatial_shapes.dtype != torch.int64 or spatial_shapes.shape != (L, 2):
        raise RuntimeError('spatial_shapes must be int64 [L, 2]')
    if level_start_index.dtype != torch.int64 or level_start_index.shape != (L,):
        raise RuntimeError('level_start_index must be int64 [L]')
    for t in (loc, attn, spatial_shapes, level_start_index):
        if t.device != value.device:
            raise RuntimeError('all tensors must be on the same device')
    if value.dtype not in DTYPE_CODES:
        raise RuntimeError(f'unsupported dtype {value.dtype}')
    mask = check_padding_mask(value, padding_mask)
    dev = value.device
    v, lc, aw, sh, st = _contig(value, loc, attn, spatial_shapes, level_start_index)
    out = torch.empty((B, Q, HD), dtype=value.dtype, device=dev)
    if out.numel() == 0:
        return out
    _check(lib_.td_layer_sample_forward(DTYPE_CODES[value.dtype], v.data_ptr(), sh.data_ptr(), st.data_ptr(),
                                        lc.data_ptr(), aw.data_ptr(), _ptr(mask), out.data_ptr(), B, Q, N, H, HD // H,
                                        L, P, _stream(dev)))
    return out


# ---- measurement kernels (not part of the operator; the benchmark's calibration) ----------------------------------

def probe_empty(launches, device=None):
    """`launches` launches of an empty kernel on the current stream of `device` (td_probe_empty)."""
    lib_ = _require()
    dev = torch.device('cuda', torch.cuda.current_device()) if device is None else torch.device(device)
    _check(lib_.td_probe_empty(launches, _stream(dev)))


def probe_gather(buf, row_bytes, loads_per_lane, workgroups, waves, sink):
    """One launch of the random-row gather probe over the bytes of `buf` (td_probe_gather); returns the bytes it
    reads. sink: an int32 tensor of at least `workgroups` elements on the same device."""
    lib_ = _require()
    if not buf.is_cuda or not buf.is_contiguous() or sink.device != buf.device or sink.numel() < workgroups or \
            sink.element_size() != 4:
        raise RuntimeError('probe_gather: contiguous device buffer and a 32-bit sink of one word per workgroup')
    nbytes = buf.numel() * buf.element_size()
    _check(lib_.td_probe_gather(buf.data_ptr(), nbytes, row_bytes, loads_per_lane, workgroups, waves,
                                sink.data_ptr(), _stream(buf.device)))
    return workgroups * waves * 64 * loads_per_lane * 16


def probe_atomic(buf, lanes, adds_per_group, workgroups, random=True):
    """One launch of the float-atomic probe over the float32 tensor `buf` (td_probe_atomic); returns the number of
    lane-group adds (each to one chunk of lanes * 4 bytes)."""
    lib_ = _require()
    if not buf.is_cuda or not buf.is_contiguous() or buf.dtype != torch.float32:
        raise RuntimeError('probe_atomic: a contiguous float32 device buffer')
    _check(lib_.td_probe_atomic(buf.data_ptr(), buf.numel() * 4, lanes, adds_per_group, workgroups, 1 if random else 0,
                                _stream(buf.device)))
    return workgroups * (256 // lanes) * adds_per_group


# ---- launch plans (the kernels' size rules, evaluated without launching; no device needed) -----------------------

def fused_plan(dtype, B, Q, N, C, H, D, L, P, aligned=True):
    """td_fused_plan: [kernel (0 vector, 1 generic, -1 none), workgroups, wavefronts per workgroup, rows per
    workgroup, balanced slices per head (0: query tiles), rows of the largest workgroup, corner groups per row,
    corner loads in flight per lane]."""
    lib_ = _require()
    out = (ctypes.c_int64 * 8)()
    _check(lib_.td_fused_plan(DTYPE_CODES[dtype], B, Q, N, C, H, D, L, P, 1 if aligned else 0, out))
    return list(out)


def sample_plan(dtype, B, Q, N, H, D, L, P, head_major=False, aligned=True):
    """td_sample_plan: [workgroups (-1: none), wavefronts per workgroup, rows per workgroup, corner groups per row,
    elements per load, 1 for rows in (b, h, q) order, corner loads in flight per lane, 0]."""
    lib_ = _require()
    out = (ctypes.c_int64 * 8)()
    _check(lib_.td_sample_plan(DTYPE_CODES[dtype], B, Q, N, H, D, L, P, 1 if head_major else 0,
                               1 if aligned else 0, out))
    return list(out)

