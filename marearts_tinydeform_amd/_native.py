"""ctypes binding of libtinydeform.so (C ABI: include/tinydeform.h) and the tensor-level host entries.

fused_forward / sample_forward / value_proj take torch tensors on a HIP device, check them the way the reference's
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
}

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
        fn = getattr(lib, name)
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
