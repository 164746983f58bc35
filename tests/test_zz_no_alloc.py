"""td_project_forward_noalloc (the project path with its projected values in the library's static per-GPU scratch
array instead of a caller workspace) against td_project_forward, through the C ABI: bit-identical outputs on two
calls in a row, the second smaller than the first (the array keeps the first call's values, which the second must
not read), in both value layouts, under HIP graph capture, and the size limit."""

import numpy as np
import pytest
import torch

from marearts_tinydeform_amd import _native
from oracle import bruteforce
from inputs import RTDETR_LEVELS, make, to, workload

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)


def both(args):
    with torch.inference_mode():
        a = _native.project_forward(*args)
        b = _native.project_forward_noalloc(*args)
    torch.cuda.synchronize()
    return a, b


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
def test_noalloc_matches_project_forward_twice(dtype):
    # float16 / bfloat16 at D = 32 take the head-major value layout, float32 the token-major one
    big = workload(2, 300, 8, 32, 256, RTDETR_LEVELS, 4, dtype)
    small = make(1, 40, 4, 16, 64, [(17, 23), (9, 12)], 4, dtype=dtype, seed=3)
    for name, args in (('B2 Q300 RT-DETR', big), ('B1 Q40 narrow heads', small)):
        say(f'  noalloc {dtype} {name}')
        dev = to(args, 'cuda')
        ref_call, got = both(dev)
        assert torch.equal(got, ref_call), f'{name}: noalloc differs from td_project_forward'
        rows = np.arange(0, got.shape[0] * got.shape[1] * args[5].shape[2], 37)
        ref = bruteforce.deform_attn(*args, rows=rows)
        D = got.shape[-1] // args[5].shape[2]
        err = np.abs(got.double().cpu().numpy().reshape(-1, D)[rows] - ref)
        tol = {torch.float16: 3e-3, torch.bfloat16: 2e-2, torch.float32: 2e-5}[dtype]
        assert (err <= tol + tol * np.abs(ref)).all(), f'{name}: max |diff| {err.max():.3g}'


def test_noalloc_under_graph_capture():
    args = to(workload(1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16), 'cuda')
    with torch.inference_mode():
        eager = _native.project_forward(*args)
        out = torch.empty_like(eager)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            _native.project_forward_noalloc(*args, out=out)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _native.project_forward_noalloc(*args, out=out)
        for i in range(4):
            out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f'graph replay {i} differs from td_project_forward'
            _native.project_forward(*args).sum().item()  # eager work between replays


def test_noalloc_refuses_problems_beyond_the_scratch_array():
    # 2 x 40000 tokens x 512 channels in float16 = 78 MB of projected values > 64 MiB: refused, nothing launched
    args = to(make(2, 8, 8, 64, 64, [(200, 200)], 2, dtype=torch.float16), 'cuda')
    w = torch.randn(512, 64, device='cuda').half()
    args[1], args[2] = w, None
    with pytest.raises(RuntimeError, match='scratch'):
        with torch.inference_mode():
            _native.project_forward_noalloc(*args)
    # just inside the limit still runs: 2 x 40000 x 256 float16 = 41 MB
    args[1] = w[:256].contiguous()
    with torch.inference_mode():
        a = _native.project_forward(*args)
        b = _native.project_forward_noalloc(*args)
    assert torch.equal(a, b)
