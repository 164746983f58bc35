"""HIP kernels vs the float64 oracle on seeded inputs (GPU). Mirrors the reference's differential tests
(tests/test_correctness.py:46-146) and adds the benchmark configurations at full size.

Tolerances: float32 atol 2e-5 / rtol 1e-4 and float16 3e-3 / bfloat16 2e-2 (atol = rtol) against float64, as the
reference's tests use (tests/test_correctness.py:70,76); float64 1e-10. At the benchmark configurations the
operator's accuracy bar holds as well, literally: max |got - ref| <= 1e-4 in float32, and
max |got - ref| / max |ref| <= 2e-2 in float16 and bfloat16 (float32 also <= 1e-4 relative).
"""

import os
import sys

import numpy as np
import pytest
import torch

import marearts_tinydeform_amd as td
from marearts_tinydeform_amd import _native
from oracle import bruteforce
import gemm_cases
from inputs import CASES, DINO_LEVELS, LIMIT_LEVELS, RTDETR_LEVELS, as_f64, make, to, workload

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (2e-5, 1e-4), torch.float16: (3e-3, 3e-3), torch.bfloat16: (2e-2, 2e-2),
       torch.float64: (1e-10, 1e-10)}
REL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2, torch.float64: 1e-10}
ABS_MAX = {torch.float32: 1e-4, torch.float64: 1e-10}  # max abs error at the benchmark configurations
MODES = ('fused', 'project', 'auto')


def say(msg):
    print(msg, flush=True)


def run(args, mode):
    with torch.inference_mode():
        out = td.ma_deform_attn(*args, mode=mode)
    torch.cuda.synchronize()
    return out


def assert_close(name, got, ref, atol, rtol):
    got = got.double().cpu().numpy() if hasattr(got, 'cpu') else got
    assert got.shape == ref.shape, f'{name}: shape {got.shape} != {ref.shape}'
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    assert not bad.any(), (f'{name}: {int(bad.sum())} elements out of tolerance, max |diff| {err.max():.3g} '
                           f'(max |ref| {np.abs(ref).max():.3g})')
    return float(err.max()) if err.size else 0.0


def check_modes(name, cpu_args, dtype, modes=MODES):
    ref = bruteforce.deform_attn(*cpu_args)
    dev = to(cpu_args, 'cuda')
    atol, rtol = TOL[dtype]
    for mode in modes:
        say(f'  {name} [{mode}]')
        assert_close(f'{name} [{mode}]', run(dev, mode), ref, atol, rtol)


def test_native_library_is_loaded():
    assert _native.lib is not None, _native.load_error
    assert os.path.dirname(_native.lib._name) == os.path.dirname(os.path.abspath(td.__file__))
    assert torch.cuda.is_available()
    say(f'device {torch.cuda.get_device_name()} arch {torch.cuda.get_device_properties(0).gcnArchName}')


@pytest.mark.parametrize('bias', [True, False])
def test_float32_cases(bias):
    for name, *shape in CASES:
        check_modes(f'{name} fp32 bias={bias}', make(*shape, bias=bias), torch.float32)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_half_and_bfloat16_cases(dtype):
    for name, *shape in CASES:
        check_modes(f'{name} {dtype}', make(*shape, dtype=dtype), dtype)


def test_float64_cases():
    for name, *shape in CASES[3:]:
        check_modes(f'{name} fp64', make(*shape, dtype=torch.float64), torch.float64)


def test_float64_fused_c8192():
    # the widest rows fused mode accepts (C <= 8192, reference csrc/ma_deform_fused.cu:301): in float64 one row of
    # accumulators takes 64 KB of LDS, beyond the default budget of a launch
    args = make(1, 6, 2, 8, 8192, [(4, 5), (2, 3)], 2, dtype=torch.float64)
    check_modes('fp64 C8192', args, torch.float64, modes=('fused', 'auto'))


def test_unaligned_memory_uses_generic_kernel():
    # reference tests/test_correctness.py:83-95: memory 2 or 4 bytes off a 16-byte boundary
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        args = make(1, 40, 8, 32, 256, [(20, 20), (10, 10)], 4, dtype=dtype)
        ref = bruteforce.deform_attn(*args)
        mem = args[0].cuda()
        buf = torch.empty(mem.numel() + 1, dtype=dtype, device='cuda')
        shifted = buf[1:].view(mem.shape)
        shifted.copy_(mem)
        assert shifted.is_contiguous() and shifted.data_ptr() % 16 != 0
        dev = [shifted] + to(args[1:], 'cuda')
        atol, rtol = TOL[dtype]
        for mode in MODES:
            say(f'  unaligned {dtype} [{mode}]')
            assert_close(f'unaligned {dtype} [{mode}]', run(dev, mode), ref, atol, rtol)


def test_far_outside_and_empty():
    # reference tests/test_correctness.py:98-106
    args = make(2, 20, 4, 8, 32, [(9, 11), (5, 6)], 4, spread=200.0)
    ref = bruteforce.deform_attn(*args)
    dev = to(args, 'cuda')
    for mode in MODES:
        assert_close(f'far outside [{mode}]', run(dev, mode), ref, 1e-5, 1e-4)
    # every sample outside: exactly zero, bias included
    allout = list(args)
    allout[5] = torch.full_like(args[5], 7.0)
    dev = to(allout, 'cuda')
    for mode in MODES:
        out = run(dev, mode)
        assert torch.count_nonzero(out) == 0, mode
    empty = to(make(1, 0, 4, 8, 32, [(9, 11)], 4), 'cuda')
    for mode in MODES:
        assert run(empty, mode).shape == (1, 0, 32)


def test_nonfinite_locations_sample_nothing():
    # clamp-before-convert rule (reference csrc/ma_deform_fused.cu:87-89): inf, -inf and NaN coordinates and
    # huge finite ones contribute nothing and never overflow the integer conversion
    for dtype in (torch.float32, torch.float16, torch.bfloat16):
        args = make(1, 16, 2, 16, 32, [(7, 9), (4, 5)], 2, dtype=dtype)
        loc = args[5].clone()
        loc[0, 0, :, :, :, 0] = float('inf')
        loc[0, 1, :, :, :, 1] = float('-inf')
        loc[0, 2, :, 0, 0, 0] = float('nan')
        loc[0, 3, :, :, :, :] = 3e4 if dtype == torch.float16 else 1e30
        args[5] = loc
        ref = bruteforce.deform_attn(*args)
        assert np.isfinite(ref).all()
        assert np.abs(ref[0, 0]).max() == 0 and np.abs(ref[0, 3]).max() == 0
        dev = to(args, 'cuda')
        atol, rtol = TOL[dtype]
        for mode in MODES:
            assert_close(f'nonfinite {dtype} [{mode}]', run(dev, mode), ref, atol, rtol)


def test_float16_sums_beyond_the_half_range():
    # un-normalised attention (about 8 per sample instead of 1 / (L P)) on memory values of about 1e4: the gathered
    # sums g pass the float16 range (65504), while the projected outputs, with a weight scaled by 1/32, stay inside
    # it. float32 accumulation, as in the reference, gives finite outputs; so must the float16 kernels.
    args = make(1, 64, 8, 32, 256, [(20, 20), (10, 10)], 4, dtype=torch.float32, spread=0.3)
    args[0] = (args[0] * 1e4).clamp(-6e4, 6e4)
    args[1] = args[1] / 32
    args[6] = args[6] * 8
    args = [t if t is None or t.dtype == torch.long else t.half() for t in args]
    ref = bruteforce.deform_attn(*args)
    g = bruteforce.deform_attn(args[0], torch.eye(256).half(), None, *args[3:])  # W = I: g itself (per head)
    assert np.abs(g).max() > 65504 and np.abs(ref).max() < 3e4
    dev = to(args, 'cuda')
    for mode in MODES:
        out = run(dev, mode)
        assert torch.isfinite(out).all(), mode
        # tolerances scaled with the values (project mode rounds its ~300-sized values to float16 on the way)
        scale = np.abs(ref).max()
        err = assert_close(f'float16 large sums [{mode}]', out, ref, 3e-3 * scale, 3e-3)
        assert err / scale <= 2e-2


def test_rejects_bad_input():
    # reference tests/test_correctness.py:109-146 (project mode checks the weight too here: our GEMM, not F.linear)
    args = to(make(1, 8, 2, 8, 16, [(6, 7), (3, 4)], 2), 'cuda')
    bad = [
        ('weight cols', 1, args[1][:, :8].contiguous()),
        ('dtype', 1, args[1].half()),
        ('bias size', 2, args[2][:4]),
        ('shapes dtype', 3, args[3].int()),
        ('starts dtype', 4, args[4].int()),
        ('too many points', 6, torch.ones(1, 8, 2, 2, 40, device='cuda') / 80),
        ('attn shape', 6, torch.ones(1, 8, 2, 2, 3, device='cuda')),
        ('loc dtype', 5, args[5].double()),
        ('batch', 0, args[0][:0]),
    ]
    for what, i, value in bad:
        a = list(args)
        a[i] = value
        if what == 'too many points':
            a[5] = torch.rand(1, 8, 2, 2, 40, 2, device='cuda')
        for mode in ('fused', 'project'):
            with pytest.raises(RuntimeError):
                with torch.inference_mode():
                    td.ma_deform_attn(*a, mode=mode)
    grad = [t.clone().requires_grad_(True) if i == 0 else t for i, t in enumerate(args)]
    with pytest.raises(RuntimeError):
        td.ma_deform_attn(*grad)
    with pytest.raises(ValueError):
        td.ma_deform_attn(*args, mode='nope')
    with pytest.raises(RuntimeError):  # C > 8192 in fused mode
        big = to(make(1, 2, 1, 8, 8200, [(2, 2)], 1, bias=False), 'cuda')
        with torch.inference_mode():
            td.ma_deform_attn(*big, mode='fused')


GEMM_EPS = {torch.float16: 2e-3, torch.bfloat16: 1e-2, torch.float32: 1e-5, torch.float64: 1e-12}


def shifted(t, offset_bytes):
    """A contiguous copy of t on the device whose data pointer lies offset_bytes past a 256-byte boundary."""
    e = t.element_size()
    assert offset_bytes % e == 0
    buf = torch.empty(t.numel() + 256 // e, dtype=t.dtype, device='cuda')
    v = buf[offset_bytes // e:offset_bytes // e + t.numel()].view(t.shape)
    v.copy_(t)
    assert v.data_ptr() % 256 == offset_bytes
    return v


def gemm_case(dt, M, K, NO, bias, offsets, kern, seed, rows=None):
    """value_proj on an [M, K] x [NO, K]^T problem whose operands sit at the given byte offsets; checks that the
    library picks kernel `kern`, then the result against the float64 oracle (on `rows`, or every row)."""
    g = torch.Generator().manual_seed(seed)
    mem = torch.randn(1, M, K, generator=g).to(dt)
    w = (torch.randn(NO, K, generator=g) / K ** 0.5).to(dt)
    b = (torch.randn(NO, generator=g) * 0.1).to(dt) if bias else None
    offsets = offsets or {}
    assert _native.value_proj_plan(dt, M, K, NO, bias=bias, offsets=offsets) == kern
    say(f'  value_proj {dt} M={M} K={K} NO={NO} bias={bias} offsets={offsets} kernel {kern}')
    dm = shifted(mem.cuda(), offsets.get('memory', 0))
    dw = shifted(w.cuda(), offsets.get('weight', 0))
    db = None if b is None else shifted(b.cuda(), offsets.get('bias', 0))
    with torch.inference_mode():
        got = _native.value_proj(dm, dw, db).cpu()
    if rows is None:
        ref = bruteforce.project(mem, w, b)
    else:
        ref = bruteforce.project(mem[:, rows], w, b)
        got = got[:, rows]
    assert_close(f'value_proj {dt} {(M, K, NO)} kernel {kern}', got, ref, GEMM_EPS[dt], GEMM_EPS[dt])


def sample_rows(M, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.cat([torch.arange(0, min(M, 300)), torch.randint(0, M, (700,), generator=g),
                      torch.arange(max(M - 300, 0), M)]).unique()


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32, torch.float64])
def test_value_proj_matches_oracle(dtype):
    # the GEMM alone, with M, N, K off the tile sizes; every row
    for (B, N, C, HD), kern in gemm_cases.SMALL:
        gemm_case(dtype, B * N, C, HD, True, None, kern[dtype], 3)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_value_proj_deep_k_matches_oracle(dtype):
    # 16-bit, K >= 512: register tiles for the small grids, both operands through LDS (9) in the middle, the
    # direct-to-LDS kernels, 256 x 128 tiles (14) and persistent 256 x 256 tiles (18) from 120 of them (one to four
    # tiles per workgroup, the last token and channel tiles moved back to overlap their neighbours), with M and the
    # output width off the tile sizes. Rows are checked on a sample that includes the first and the last M tile.
    for M, K, NO, kern in gemm_cases.DEEP_K:
        gemm_case(dtype, M, K, NO, True, None, kern, 11, rows=sample_rows(M, 11))


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_value_proj_streaming_matches_oracle(dtype):
    # 16-bit, 256 outputs, K = 128 or 256, from 14000 / 8000 rows: the streaming kernel (W resident in registers,
    # tokens streamed through LDS; each workgroup an equal share of the rows); see tests/gemm_cases.py for the step
    # structure each M takes. Every row is checked: the share boundaries fall anywhere in M. Odd M, with and without
    # bias.
    for M, K, bias, kern in gemm_cases.STREAM:
        gemm_case(dtype, M, K, 256, bias, None, kern, 12)


def test_value_proj_unaligned_bias_falls_back():
    # a bias view 2 bytes off a 16-byte boundary (buf[1:] in float16) at sizes the streaming kernel would take
    for M, K, NO, kern in gemm_cases.BIAS_OFFSET:
        gemm_case(torch.float16, M, K, NO, True, {'bias': 2}, kern, 13)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
def test_value_proj_unaligned_operands_use_generic_kernel(dtype):
    for M, K, NO, offsets, kern in gemm_cases.UNALIGNED:
        gemm_case(dtype, M, K, NO, True, offsets, kern, 14)


def heads_of(value, H):
    """[B, N, H * D] -> head-major [B, H, N, D] (torch tensor or numpy array)."""
    B, N, HD = value.shape
    if isinstance(value, np.ndarray):
        return np.ascontiguousarray(value.reshape(B, N, H, HD // H).transpose(0, 2, 1, 3))
    return value.reshape(B, N, H, HD // H).permute(0, 2, 1, 3).contiguous()


def test_value_proj_heads_matches_oracle():
    # the head-major GEMM output: row b * N + t, column h * D + d lands at [b, h, t, d]. The shapes reach every tile
    # family (tests/gemm_cases.py), with ragged B, N and heads of 16 bytes. Every row is checked.
    g = torch.Generator().manual_seed(21)
    for dtype, cases in gemm_cases.HEADS.items():
        for (B, N, C, H, D), kern in cases:
            say(f'  value_proj_heads {dtype} B={B} N={N} C={C} H={H} D={D} kernel {kern}')
            assert _native.value_proj_plan(dtype, B * N, C, H * D, heads=H, N=N) == kern
            mem = torch.randn(B, N, C, generator=g).to(dtype)
            w = (torch.randn(H * D, C, generator=g) / C ** 0.5).to(dtype)
            b = (torch.randn(H * D, generator=g) * 0.1).to(dtype)
            with torch.inference_mode():
                got = _native.value_proj_heads(mem.cuda(), w.cuda(), b.cuda(), H).cpu()
            assert got.shape == (B, H, N, D)
            ref = heads_of(bruteforce.project(mem, w, b), H)
            assert_close(f'value_proj_heads {dtype} {(B, N, C, H, D)}', got, ref, GEMM_EPS[dtype], GEMM_EPS[dtype])


def test_sample_heads_matches_oracle():
    # the sampler on a head-major value: same results as on [B, N, H * D] (every case, every dtype; any D)
    for dtype in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        for name, B, Q, H, D, C, levels, P in CASES:
            args = make(B, Q, H, D, C, levels, P, dtype=dtype)
            g = torch.Generator().manual_seed(6)
            value = torch.randn(B, args[0].shape[1], H * D, generator=g).to(dtype)
            ref = bruteforce.sample(value, H, *args[3:])
            with torch.inference_mode():
                got = _native.sample_forward_heads(heads_of(value, H).cuda(), *to(args[3:], 'cuda'))
            torch.cuda.synchronize()
            atol, rtol = TOL[dtype]
            assert_close(f'sample_heads {name} {dtype}', got, ref, atol, rtol)


def test_sample_alone_matches_oracle():
    for dtype in (torch.float16, torch.bfloat16, torch.float32):
        for name, B, Q, H, D, C, levels, P in CASES:
            args = make(B, Q, H, D, C, levels, P, dtype=dtype)
            g = torch.Generator().manual_seed(5)
            value = torch.randn(B, args[0].shape[1], H * D, generator=g).to(dtype)
            ref = bruteforce.sample(value, H, *args[3:])
            with torch.inference_mode():
                got = td.ma_deform_sample(value.cuda(), *to(args[3:], 'cuda'))
            torch.cuda.synchronize()
            atol, rtol = TOL[dtype]
            assert_close(f'sample {name} {dtype}', got, ref, atol, rtol)


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32])
def test_sample_head_order_on_large_values(dtype):
    # values of 44.6 MB (fp16) / 89 MB (fp32) per image, each head's rows read about twice (4 Q L P / N = 2.01): the
    # sampler takes its rows head by head ((b, h, q) order) instead of in the output's (b, q, h) order; two images, a
    # query count that tiles nothing, a padding mask on the second call. Token-major and head-major values.
    B, Q, H, D, P = 2, 171, 16, 64, 16
    args = make(B, Q, H, D, H * D, LIMIT_LEVELS, P, dtype=dtype)
    N = args[0].shape[1]
    g = torch.Generator().manual_seed(9)
    value = torch.randn(B, N, H * D, generator=g).to(dtype)
    mask = torch.rand(B, N, generator=g) < 0.2
    ref = bruteforce.sample(value, H, *args[3:])
    ref_m = bruteforce.sample(value, H, *args[3:], padding_mask=mask)
    dev = to(args[3:], 'cuda')
    with torch.inference_mode():
        got = td.ma_deform_sample(value.cuda(), *dev)
        got_m = td.ma_deform_sample(value.cuda(), *dev, padding_mask=mask.cuda())
        got_h = _native.sample_forward_heads(heads_of(value, H).cuda(), *dev)
    torch.cuda.synchronize()
    atol, rtol = TOL[dtype]
    assert_close(f'sample (b, h, q) order {dtype}', got, ref, atol, rtol)
    assert_close(f'sample (b, h, q) order, mask {dtype}', got_m, ref_m, atol, rtol)
    assert_close(f'sample_heads (b, h, q) order {dtype}', got_h, ref, atol, rtol)


def big_memory_case(name, dtype, Q, tokens, masked):
    """One image whose memory has `tokens` C-wide rows: filler levels of zero rows (a 2048-wide map, then a one-row
    map for the remainder) whose samples carry weight 0, and a 32 x 32 level of random rows at the tensor's end. The
    result is that of the last level alone, which the oracle computes on the small problem. Query 0 samples the
    last token of the tensor in every head (bilinear x0 = y0 = 31), so the last rows are read whichever way the
    kernels address them. With `masked`, a padding mask over a fifth of the small level's tokens (and none of the
    filler) makes the kernels take their general corner rule."""
    B, H, D, C, P, small = 1, 8, 32, 256, 4, (32, 32)
    N1 = small[0] * small[1]
    fill = tokens - N1
    h0 = fill // 2048
    levels = [(h0, 2048)] + ([(1, fill - h0 * 2048)] if fill > h0 * 2048 else [])
    LF = len(levels)
    args = make(B, Q, H, D, C, [small], P, dtype=dtype)
    mem1, w, b, _, _, loc1, attn1 = args
    loc1[0, 0, :, 0, 0] = 1 - 0.25 / 32   # x = y = 31.25: corner (31, 31) is the last token
    loc1[0, 0, :, 0, 1] = 1.0             # x = y = 31.5
    args[5] = loc1
    g = torch.Generator().manual_seed(17)
    mask1 = torch.rand(B, N1, generator=g) < 0.2 if masked else None
    loc0 = torch.rand(B, Q, H, LF, P, 2, generator=g).to(dtype)
    loc = torch.cat([loc0, loc1], dim=3)
    attn = torch.cat([torch.zeros(B, Q, H, LF, P, dtype=dtype), attn1], dim=3)
    ref = bruteforce.deform_attn(*args, padding_mask=mask1)
    memory = torch.zeros(B, tokens, C, dtype=dtype, device='cuda')
    memory[:, fill:] = mem1.cuda()
    shapes = torch.tensor(levels + [small], dtype=torch.int64, device='cuda')
    starts = torch.tensor([0, h0 * 2048, fill][:LF + 1], dtype=torch.int64, device='cuda')
    mask = None
    if masked:
        mask = torch.zeros(B, tokens, dtype=torch.bool, device='cuda')
        mask[:, fill:] = mask1.cuda()
    dev = [memory, w.cuda(), b.cuda(), shapes, starts, loc.cuda(), attn.cuda()]
    atol, rtol = TOL[dtype]
    for mode in ('fused', 'project'):
        say(f'  {name} {dtype} Q{Q} tokens {tokens} ({tokens * C * memory.element_size()} bytes)'
            f'{" masked" if masked else ""} [{mode}]')
        with torch.inference_mode():
            out = td.ma_deform_attn(*dev, mode=mode, padding_mask=mask)
        torch.cuda.synchronize()
        assert_close(f'{name} {dtype} Q{Q} [{mode}]', out.double().cpu().numpy(), ref, atol, rtol)
    del memory, dev, mask
    torch.cuda.empty_cache()


@pytest.mark.parametrize('dtype,Q,masked', [
    (torch.float16, 16, False),    # 128 rows: two-wavefront balanced slices; head-major sampler
    (torch.bfloat16, 16, False),
    (torch.float32, 16, False),    # token-major sampler (float32 head rows of 128 bytes)
    (torch.float16, 1024, False),  # 8192 rows: 8-wavefront query tiles
    (torch.bfloat16, 16, True),    # padding mask: the general corner rule's kernels
])
def test_tensors_of_2gb_take_the_64bit_gather(dtype, Q, masked):
    # Memory and value tensors of 2 GB or more are gathered with 64-bit addresses instead of 32-bit buffer offsets
    # (memory and value have the same bytes here: H * D = C).
    row = 256 * torch.empty(0, dtype=dtype).element_size()
    tokens = 2 ** 31 // row + 1024
    assert tokens * row >= 2 ** 31
    big_memory_case('2 GB memory', dtype, Q, tokens, masked)


@pytest.mark.parametrize('dtype', [torch.float16, torch.float32])
def test_tensors_just_under_2gb_keep_the_buffer_gather(dtype):
    # 4 KB short of 2^31 bytes: the buffer-load gathers at the top of their range, where the last rows' offsets
    # t * row + lane offset come closest to the outside corners' 2^31.
    row = 256 * torch.empty(0, dtype=dtype).element_size()
    tokens = (2 ** 31 - 4096) // row
    assert (tokens + 1) * row > 2 ** 31 - 4096 and tokens * row < 2 ** 31
    big_memory_case('memory under 2 GB', dtype, 16, tokens, False)


def test_graph_capture_replays_match_eager():
    args = to(workload(1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16), 'cuda')
    for mode in MODES:
        with torch.inference_mode():
            eager = td.ma_deform_attn(*args, mode=mode)
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(2):
                    td.ma_deform_attn(*args, mode=mode)
            torch.cuda.current_stream().wait_stream(s)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                out = td.ma_deform_attn(*args, mode=mode)
            for i in range(4):
                out.zero_()
                torch.cuda.synchronize()
                graph.replay()
                torch.cuda.synchronize()
                assert torch.equal(out, eager), f'graph replay {i} [{mode}] differs from eager'
                _ = eager.sum().item()  # eager work between replays


# ---- the benchmark configurations at full size ---------------------------------------------------------------

def full_size_check(name, args, dtype, rows=None, modes=('fused', 'project')):
    H = args[5].shape[2]
    B, Q = args[5].shape[:2]
    if rows is None:
        ref = bruteforce.deform_attn(*args)
    else:
        ref = bruteforce.deform_attn(*args, rows=rows)
    dev = to(args, 'cuda')
    atol, rtol = TOL[dtype]
    outs = {}
    for mode in modes:
        say(f'  {name} [{mode}]')
        out = run(dev, mode)
        assert out.shape == (B, Q, args[1].shape[0])
        assert torch.isfinite(out).all()
        outs[mode] = out
        got = out.double().cpu().numpy()
        if rows is not None:
            D = got.shape[-1] // H
            got = got.reshape(-1, D)[rows]
        err = assert_close(f'{name} [{mode}]', got, ref, atol, rtol)
        rel = err / max(np.abs(ref).max(), 1e-30)
        say(f'    max |diff| {err:.3g}, relative {rel:.3g}')
        assert rel <= REL[dtype], f'{name} [{mode}]: relative error {rel:.3g}'
        if dtype in ABS_MAX:
            assert err <= ABS_MAX[dtype], f'{name} [{mode}]: max abs error {err:.3g}'
    if len(outs) == 2:  # linear reordering: both orders agree over the whole output
        a, b = (o.double() for o in outs.values())
        assert torch.allclose(a, b, atol=2 * atol, rtol=2 * rtol), f'{name}: fused and project disagree'


@pytest.mark.parametrize('Q', [50, 100, 300])
def test_rtdetr640_fp16_b1(Q):
    full_size_check(f'rtdetr640 fp16 B1 Q{Q}', workload(1, Q, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16),
                    torch.float16)


@pytest.mark.parametrize('dtype,B,Q', [
    (torch.float16, 1, 150),    # rows gathered by two wavefronts, one 12-wavefront slice per CU
    (torch.bfloat16, 1, 150),
    (torch.float16, 2, 300),    # one wavefront per row, two 12-wavefront slices per CU
    (torch.float32, 2, 300),
    (torch.float16, 3, 300),    # four 8-wavefront slices per CU, 6 loads in flight per lane
    (torch.bfloat16, 3, 300),
    (torch.float16, 4, 50),     # one 8-wavefront slice of 7 rows per CU
])
def test_rtdetr640_slice_shapes(dtype, B, Q):
    # the fused kernel's balanced-slice launch shapes beyond the benchmark configurations (sampled rows against the
    # oracle, fused and project over the whole output)
    rows = np.sort(np.random.default_rng(B * Q).choice(B * Q * 8, size=min(B * Q * 8, 1536), replace=False))
    full_size_check(f'rtdetr640 {dtype} B{B} Q{Q}', workload(B, Q, 8, 32, 256, RTDETR_LEVELS, 4, dtype), dtype,
                    rows=rows)


@pytest.mark.parametrize('dtype,B,Q', [(torch.float16, 1, 450), (torch.bfloat16, 2, 150), (torch.float32, 1, 300),
                                        (torch.float16, 5, 150)])
def test_wide_rows_c768(dtype, B, Q):
    # C = 768 (12 heads of 64): rows wider than a wavefront (96 lanes in 16 bits, 192 in float32) that do not tile
    # four wavefronts, gathered by 12-wavefront workgroups for small problems and 8-wavefront ones from 8192 rows;
    # sampled rows against the oracle, fused and project over the whole output
    rows = np.sort(np.random.default_rng(B * Q + 1).choice(B * Q * 12, size=min(B * Q * 12, 1536), replace=False))
    full_size_check(f'c768 {dtype} B{B} Q{Q}', workload(B, Q, 12, 64, 768, RTDETR_LEVELS, 4, dtype), dtype, rows=rows)


def test_rtdetr640_fp32_b1_q300():
    full_size_check('rtdetr640 fp32 B1 Q300', workload(1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float32),
                    torch.float32)


def test_rtdetr640_bf16_b8_q300():
    full_size_check('rtdetr640 bf16 B8 Q300', workload(8, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.bfloat16),
                    torch.bfloat16)


def test_dino_4level_fp16_b4_q900():
    full_size_check('dino fp16 B4 Q900',
                    workload(4, 900, 8, 32, 256, DINO_LEVELS, 4, torch.float16, loc_dist='outside10'),
                    torch.float16)


def test_dino_encoder_fp16_b2():
    # encoder self-attention: every memory token is a query (Q = N = 22223), sampling around its own position;
    # 2048 sampled rows against the oracle, fused and project compared over the whole output
    args = workload(2, 22223, 8, 32, 256, DINO_LEVELS, 4, torch.float16, loc_dist='encoder')
    rows = np.random.default_rng(7).choice(2 * 22223 * 8, size=2048, replace=False)
    full_size_check('dino encoder fp16 B2 Q=N', args, torch.float16, rows=np.sort(rows))


@pytest.mark.parametrize('Q', [50, 300, 900])
def test_limit_case_bf16_c1024(Q):
    args = workload(2, Q, 16, 64, 1024, LIMIT_LEVELS, 16, torch.bfloat16, bias=False)
    rows = np.random.default_rng(Q).choice(2 * Q * 16, size=min(1024, 2 * Q * 16), replace=False)
    full_size_check(f'limit bf16 C1024 B2 Q{Q}', args, torch.bfloat16, rows=np.sort(rows))


def test_limit_case_bf16_c1024_b1_project():
    # the C = 1024 limit shape at batch 1 (21760 tokens: the persistent 256 x 256 direct-to-LDS value GEMM, 340 tiles
    # on 256 workgroups), project mode end to end, 1024 sampled rows against the oracle
    args = workload(1, 300, 16, 64, 1024, LIMIT_LEVELS, 16, torch.bfloat16, bias=False)
    assert _native.value_proj_plan(torch.bfloat16, 21760, 1024, 1024, bias=False, heads=16, N=21760) == 18
    rows = np.random.default_rng(1).choice(300 * 16, size=1024, replace=False)
    full_size_check('limit bf16 C1024 B1 Q300', args, torch.bfloat16, rows=np.sort(rows), modes=('project',))


# ---- value padding mask ---------------------------------------------------------------------------------------

def padded_images_mask(B, levels, seed):
    """Padding as a batch of different-size images produces: per image and level, the right and bottom part of
    the map is padding (True)."""
    g = torch.Generator().manual_seed(seed)
    masks = []
    for b in range(B):
        keep_w, keep_h = 0.5 + 0.5 * torch.rand(2, generator=g).tolist()[0], 0.5 + 0.5 * torch.rand(1, generator=g).item()
        per_level = []
        for h, w in levels:
            m = torch.zeros(h, w, dtype=torch.bool)
            m[:, max(1, int(round(w * keep_w))):] = True
            m[max(1, int(round(h * keep_h))):, :] = True
            per_level.append(m.flatten())
        masks.append(torch.cat(per_level))
    return torch.stack(masks)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
def test_padding_mask_cases(dtype):
    for name, B, Q, H, D, C, levels, P in CASES:
        args = make(B, Q, H, D, C, levels, P, dtype=dtype)
        mask = torch.rand(B, args[0].shape[1], generator=torch.Generator().manual_seed(7)) < 0.3
        ref = bruteforce.deform_attn(*args, padding_mask=mask)
        dev = to(args, 'cuda')
        atol, rtol = TOL[dtype]
        for mode in MODES:
            with torch.inference_mode():
                out = td.ma_deform_attn(*dev, mode=mode, padding_mask=mask.cuda())
            assert_close(f'mask {name} {dtype} [{mode}]', out, ref, atol, rtol)
        # sampling alone on projected values
        value = bruteforce.project(args[0], args[1], args[2])
        vdev = torch.from_numpy(value).to(dtype).cuda()
        with torch.inference_mode():
            out = td.ma_deform_sample(vdev, *dev[3:], padding_mask=mask.cuda())
        ref_s = bruteforce.sample(vdev.double().cpu(), H, *args[3:], padding_mask=mask)
        assert_close(f'mask sample {name} {dtype}', out, ref_s, atol, rtol)


def test_padding_mask_everything_padded_is_zero():
    args = to(make(2, 9, 4, 8, 32, [(9, 11), (5, 6)], 4), 'cuda')
    mask = torch.ones(2, args[0].shape[1], dtype=torch.bool, device='cuda')
    for mode in MODES:
        with torch.inference_mode():
            out = td.ma_deform_attn(*args, mode=mode, padding_mask=mask)
        assert torch.count_nonzero(out) == 0, mode
    with pytest.raises(RuntimeError):
        td.ma_deform_attn(*args, padding_mask=mask[:, :5])


def test_padding_mask_rtdetr640_fp16_b4_padded_images():
    args = workload(4, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16)
    mask = padded_images_mask(4, RTDETR_LEVELS, 11)
    assert 0.1 < mask.float().mean() < 0.7
    ref = bruteforce.deform_attn(*args, padding_mask=mask)
    dev = to(args, 'cuda')
    atol, rtol = TOL[torch.float16]
    outs = []
    for mode in ('fused', 'project'):
        with torch.inference_mode():
            out = td.ma_deform_attn(*dev, mode=mode, padding_mask=mask.cuda())
        err = assert_close(f'padded images [{mode}]', out, ref, atol, rtol)
        assert err / np.abs(ref).max() <= REL[torch.float16]
        outs.append(out.double())
    assert torch.allclose(outs[0], outs[1], atol=2 * atol, rtol=2 * rtol)


# ---- D-FINE core: per-level point counts, discrete method ---------------------------------------------------

def dfine_case(B, Q, H, D, levels, points, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    shapes = torch.tensor(levels, dtype=torch.long)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([torch.zeros(1, dtype=torch.long), sizes.cumsum(0)[:-1]])
    N, J = int(sizes.sum()), sum(points)
    value = torch.randn(B, N, H, D, generator=g).to(dtype)
    loc = (torch.rand(B, Q, 1, 1, 2, generator=g) + 0.3 * torch.randn(B, Q, H, J, 2, generator=g)).to(dtype)
    attn = torch.randn(B, Q, H, J, generator=g).softmax(-1).to(dtype)
    return value, shapes, starts, loc, attn


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize('method', ['default', 'discrete'])
def test_dfine_sample_v2(dtype, method):
    for points, levels in (([3, 6, 3], RTDETR_LEVELS), ([4, 4, 4], RTDETR_LEVELS), ([2, 1, 5, 3], DINO_LEVELS)):
        value, shapes, starts, loc, attn = dfine_case(2, 120, 8, 32, levels, points, dtype)
        mask = torch.rand(2, value.shape[1], generator=torch.Generator().manual_seed(3)) < 0.2
        atol, rtol = TOL[dtype]
        for m in (None, mask):
            ref = bruteforce.sample_v2(value, shapes, starts, loc, attn, points, method, padding_mask=m)
            with torch.inference_mode():
                out = td.ma_deform_sample_v2(value.cuda(), shapes.cuda(), starts.cuda(), loc.cuda(), attn.cuda(),
                                             points, method, padding_mask=None if m is None else m.cuda())
            assert_close(f'dfine {points} {method} {dtype} mask={m is not None}', out, ref, atol, rtol)
    with pytest.raises(RuntimeError):  # counts that do not add up to the sample dimension
        td.ma_deform_sample_v2(value.cuda(), shapes.cuda(), starts.cuda(), loc.cuda(), attn.cuda(), [2, 2, 2, 2])
    with pytest.raises(ValueError):
        td.ma_deform_sample_v2(value.cuda(), shapes.cuda(), starts.cuda(), loc.cuda(), attn.cuda(), points, 'nope')


@pytest.mark.parametrize('dtype,B', [(torch.float16, 1), (torch.bfloat16, 1), (torch.float32, 1), (torch.bfloat16, 8)])
def test_phase_stamp_build_computes_what_the_library_computes(dtype, B):
    # bench.py --phases times libtinydeform_phases.so: the same fused kernel with stamps. Its outputs must be the
    # library's bit for bit (RT-DETR 640, Q300: one slice per CU at B1, 16-row query tiles at B8), and every
    # stamped wavefront's stamps must follow the kernel's phase order.
    import ctypes
    path = os.path.join(os.path.dirname(_native.LIB_PATH), 'libtinydeform_phases.so')
    phases = _native.load(path)
    assert phases is not None, _native.load_error
    phases.td_phase_stamps.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    phases.td_phase_stamps.restype = ctypes.c_int
    say(f'  phase build, {dtype}, B{B} Q300')
    dev = to(workload(B, 300, 8, 32, 256, RTDETR_LEVELS, 4, dtype), 'cuda')
    want = run(dev, 'fused')
    plain = _native.lib
    try:
        _native.lib = phases
        got = run(dev, 'fused')
    finally:
        _native.lib = plain
    assert torch.equal(got, want)
    n = 1024 * 12 * 16
    buf = np.zeros(n, dtype=np.uint64)
    assert phases.td_phase_stamps(buf.ctypes.data, n) == 0
    plan = _native.fused_plan(dtype, B, 300, 8400, 256, 8, 32, 3, 4)
    st = buf.reshape(1024, 12, 16)[:min(plan[1], 1024), :plan[2]].astype(np.int64)
    order = [11, 0, 1, 2, 3, 4, 8, 9, 10]  # entry .. outputs stored: every wavefront of every stamped workgroup
    seq = st[:, :, order]
    assert (seq > 0).all()
    assert (np.diff(seq, axis=-1) >= 0).all()
