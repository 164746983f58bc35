"""The backward on the GPU: gradients of ma_deform_attn_train / ma_deform_sample_train (td_sample_backward,
td_input_grad, td_weight_grad) against the float64 gradient oracle (oracle.gridsample.deform_attn_grads, pinned in
tests/test_backward.py against finite differences of the brute force).

Tolerance: the largest elementwise difference relative to the largest oracle entry of that gradient: float64
1e-10, float32 2e-4, float16 1e-2, bfloat16 3e-2. The 16-bit inputs carry their own rounding into every gradient
(the value gradient is accumulated in float32 and rounded once to the input type before the projection GEMMs, as
the forward rounds the value), and the location gradient is a difference of corner products, so the 16-bit bars
are looser than the forward's.
"""

import numpy as np
import pytest
import torch

import marearts_tinydeform_amd as td
from marearts_tinydeform_amd import _native
from oracle import gridsample
from inputs import CASES, RTDETR_LEVELS, make, to, workload

pytestmark = pytest.mark.gpu

REL = {torch.float64: 1e-10, torch.float32: 2e-4, torch.float16: 1e-2, torch.bfloat16: 3e-2}
NAMES = ('memory', 'value_weight', 'value_bias', 'sampling_locations', 'attention_weights')
POS = (0, 1, 2, 5, 6)


def say(msg):
    print(msg, flush=True)


def grad_out_for(args, seed=9):
    B, Q, H = args[5].shape[:3]
    HD = args[1].shape[0]
    return torch.randn(B, Q, HD, generator=torch.Generator().manual_seed(seed))


def gpu_grads(args, grad_out, dtype, mask=None):
    dev = [None if t is None else t.cuda() for t in args]
    leaves = [t.requires_grad_(True) if (i in POS and t is not None) else t for i, t in enumerate(dev)]
    out = td.ma_deform_attn_train(*leaves, padding_mask=None if mask is None else mask.cuda())
    out.backward(grad_out.to(dtype).cuda())
    torch.cuda.synchronize()
    return {n: None if leaves[p] is None else leaves[p].grad for n, p in zip(NAMES, POS)}, out


def boundary_distance(loc, levels):
    """The smallest distance, in pixels, of a sample's x = loc * W - 0.5 (or y) from an integer that is not 0: where
    the two coincide exactly the float32 and float64 floors agree."""
    best = float('inf')
    for l, (hl, wl) in enumerate(levels):
        for k, size in ((0, wl), (1, hl)):
            c = loc[..., l, :, k].double() * size - 0.5
            dist = (c - c.round()).abs()
            dist = dist[dist > 0]
            if dist.numel():
                best = min(best, float(dist.min()))
    return best


def check(name, got, ref, dtype):
    if ref is None:
        assert got is None, name
        return
    got = got.double().cpu().numpy()
    assert got.shape == ref.shape, f'{name}: {got.shape} != {ref.shape}'
    scale = max(float(np.abs(ref).max()), 1e-6)
    err = float(np.abs(got - ref).max()) / scale
    assert err <= REL[dtype], f'{name}: max |diff| / max |ref| = {err:.3g} > {REL[dtype]}'


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize('case', CASES, ids=[c[0] for c in CASES])
def test_gradients_match_oracle(case, dtype):
    name, B, Q, H, D, C, levels, P = case
    args = make(B, Q, H, D, C, levels, P, dtype=dtype)
    go = grad_out_for(args)
    say(f'  backward {name} {dtype}')
    grads, _ = gpu_grads(args, go, dtype)
    ref = gridsample.deform_attn_grads(*args, go.to(dtype))
    for n in NAMES:
        check(f'{name} {dtype} d{n}', grads[n], ref[n], dtype)


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
@pytest.mark.parametrize('D', [96, 128, 256])
def test_gradients_wide_heads(D, dtype):
    # head dims above 64 take the several-channels-per-lane sampling backward (D <= 64 the batched one, covered by
    # the cases above); 96 is not a power of two
    args = make(1, 20, 2, D, 64, [(10, 12), (5, 6)], 2, dtype=dtype)
    go = grad_out_for(args)
    say(f'  backward wide heads D={D} {dtype}')
    grads, _ = gpu_grads(args, go, dtype)
    ref = gridsample.deform_attn_grads(*args, go.to(dtype))
    for n in NAMES:
        check(f'D={D} {dtype} d{n}', grads[n], ref[n], dtype)


@pytest.mark.parametrize('dtype', [torch.float32, torch.bfloat16])
def test_gradients_with_padding_mask_and_no_bias(dtype):
    args = make(2, 50, 8, 32, 256, [(40, 40), (20, 20), (10, 10)], 4, dtype=dtype, bias=False)
    N = args[0].shape[1]
    mask = torch.rand(2, N, generator=torch.Generator().manual_seed(4)) < 0.3
    go = grad_out_for(args)
    grads, _ = gpu_grads(args, go, dtype, mask=mask)
    ref = gridsample.deform_attn_grads(*args, go.to(dtype), padding_mask=mask)
    for n in NAMES:
        check(f'masked d{n}', grads[n], ref[n], dtype)
    # a padded token's memory row gets no gradient
    assert not grads['memory'][mask.cuda()].any()


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16])
def test_sample_only_gradients(dtype):
    # ma_deform_sample_train: the oracle with the identity projection is the sampling alone
    name, B, Q, H, D, C, levels, P = CASES[2]
    args = make(B, Q, H, D, C, levels, P, dtype=dtype)
    value = torch.randn(B, args[0].shape[1], H * D, generator=torch.Generator().manual_seed(2)).to(dtype)
    go = grad_out_for(args)
    v = value.cuda().requires_grad_(True)
    loc = args[5].cuda().requires_grad_(True)
    attn = args[6].cuda().requires_grad_(True)
    out = td.ma_deform_sample_train(v, args[3].cuda(), args[4].cuda(), loc, attn)
    out.backward(go.to(dtype).cuda())
    eye = torch.eye(H * D, dtype=dtype)
    ref = gridsample.deform_attn_grads(value, eye, None, args[3], args[4], args[5], args[6], go.to(dtype))
    check('dvalue', v.grad, ref['memory'], dtype)
    check('dloc', loc.grad, ref['sampling_locations'], dtype)
    check('dattn', attn.grad, ref['attention_weights'], dtype)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
def test_projection_gradients_alone(dtype):
    # td_input_grad / td_weight_grad on shapes off the tile sizes, split-K included, against float64 matmuls
    g = torch.Generator().manual_seed(8)
    # (the last shape has C and H * D off the 16-byte vector width: scalar staging in the weight gradient; 1024 x 1024
    # is 64 output tiles, planned for 1024 workgroups; from C = 512 on the weight gradient's column tiles are 256 wide,
    # and C = 520 and 516 leave the last one 8 and 4 columns, with 16-byte and scalar staging; 520 x 520 and 516 x 516
    # are ragged in both the row and the column tiles)
    for (B, N, C, HD) in ((1, 8400, 256, 256), (2, 77, 40, 48), (1, 1000, 1024, 96), (3, 5, 8, 16), (1, 50, 36, 30),
                          (1, 3000, 1024, 1024), (1, 700, 520, 64), (1, 300, 516, 40), (1, 400, 520, 520),
                          (1, 300, 516, 516)):
        gv = torch.randn(B, N, HD, generator=g).to(dtype)
        mem = torch.randn(B, N, C, generator=g).to(dtype)
        w = (torch.randn(HD, C, generator=g) / C ** 0.5).to(dtype)
        say(f'  projection grads {dtype} {(B, N, C, HD)}')
        gm = _native.input_grad(gv.cuda(), w.cuda())
        gw, gb = _native.weight_grad(gv.cuda(), mem.cuda())
        torch.cuda.synchronize()
        G, X = gv.double().reshape(-1, HD), mem.double().reshape(-1, C)
        check('grad_memory', gm, (G @ w.double()).reshape(B, N, C).numpy(), dtype)
        check('grad_weight', gw, (G.T @ X).numpy(), dtype)
        check('grad_bias', gb, G.sum(0).numpy(), dtype)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16, torch.float64])
def test_input_and_weight_gradients_in_one_call(dtype):
    # td_input_weight_grad against td_input_grad and td_weight_grad, bit for bit: (1, 8400, 256, 256) and the two
    # ragged shapes (M, N and K off the tiles; C a multiple of 8 or not, so the weight gradient stages 16-byte pieces
    # or scalars) share one launch in 16/32 bits (in 16 bits with C % 8 = 0 reading W as stored); (1, 16800, 256,
    # 256) and (2, 5000, 256, 128) take the streaming GEMM, in 16 bits also with W as stored, against td_input_grad's
    # transposed copy; the others take the two kernels one after the other
    g = torch.Generator().manual_seed(12)
    for (B, N, C, HD) in ((1, 8400, 256, 256), (1, 5000, 264, 136), (1, 5000, 260, 136), (2, 77, 40, 48),
                          (1, 1000, 1024, 96), (1, 16800, 256, 256), (2, 5000, 256, 128)):
        gv = torch.randn(B, N, HD, generator=g).to(dtype).cuda()
        mem = torch.randn(B, N, C, generator=g).to(dtype).cuda()
        w = (torch.randn(HD, C, generator=g) / C ** 0.5).to(dtype).cuda()
        say(f'  input and weight gradients {dtype} {(B, N, C, HD)}')
        gm, gw, gb = _native.input_weight_grad(gv, w, mem)
        gm1 = _native.input_grad(gv, w)
        gw1, gb1 = _native.weight_grad(gv, mem)
        torch.cuda.synchronize()
        assert torch.equal(gm, gm1) and torch.equal(gw, gw1) and torch.equal(gb, gb1)
        G, X = gv.double().cpu().reshape(-1, HD), mem.double().cpu().reshape(-1, C)
        check('grad_memory', gm, (G @ w.double().cpu()).reshape(B, N, C).numpy(), dtype)
        check('grad_weight', gw, (G.T @ X).numpy(), dtype)


def test_weight_gradient_is_deterministic():
    g = torch.Generator().manual_seed(1)
    gv = torch.randn(1, 8400, 256, generator=g).half().cuda()
    mem = torch.randn(1, 8400, 256, generator=g).half().cuda()
    first = _native.weight_grad(gv, mem)
    for _ in range(3):
        again = _native.weight_grad(gv, mem)
        assert torch.equal(first[0], again[0]) and torch.equal(first[1], again[1])


def test_headline_shape_backward():
    # RT-DETR 640, B=1, Q=300, float16 (the benchmark's inputs): every gradient against the oracle
    args = workload(1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16)
    go = grad_out_for(args)
    grads, out = gpu_grads(args, go, torch.float16)
    ref = gridsample.deform_attn_grads(*args, go.half())
    for n in NAMES:
        check(f'headline d{n}', grads[n], ref[n], torch.float16)
    # the forward of the training entry is the operator's project mode
    with torch.inference_mode():
        fwd = td.ma_deform_attn(*to(args, 'cuda'), mode='project')
    assert torch.equal(out.detach(), fwd)


SORT_LEVELS = {'four': [(48, 64), (24, 32), (12, 16), (6, 8)], 'wide': [(64, 80), (32, 40), (16, 20)],
               'big': [(96, 128), (48, 64)], 'dino': [(50, 84), (25, 42), (13, 21)]}


@pytest.mark.parametrize('dtype,D,shape,Q', [(torch.float16, 32, 'four', 901), (torch.bfloat16, 32, 'four', 901),
                                             (torch.float16, 64, 'four', 901), (torch.bfloat16, 16, 'wide', 901),
                                             (torch.float16, 8, 'big', 600), (torch.bfloat16, 8, 'big', 700),
                                             (torch.bfloat16, 4, 'big', 600), (torch.float16, 32, 'dino', 400),
                                             (torch.bfloat16, 64, 'dino', 400)])
@pytest.mark.parametrize('with_mask', [False, True])
def test_decoder_sorted_value_gradients(dtype, D, shape, Q, with_mask):
    # decoder density with many corners (2^18 and more, 16-bit): the value gradient by binning the corners by token
    # (sort_count_kernel .. sort_reduce_kernel, written once in the element type) and the location and weight
    # gradients by loc_attn_backward_kernel; Q ragged against the query tiles, clustered and uniform locations.
    # Bins per level: where the scratch is tight ('four', 'wide') wide bins, the small levels' bins then split into
    # token ranges; 'dino' has room for narrow bins on its small levels (8-16 tokens), with hot spots split when
    # clustered. D = 4 (16-bit): narrower than loc_attn_backward_kernel's 16-byte loads, so the atomic scatter
    levels = SORT_LEVELS[shape]
    L, P = len(levels), 4
    N = sum(h * w for h, w in levels)
    mask = (torch.rand(2, N, generator=torch.Generator().manual_seed(5)) < 0.2) if with_mask else None
    for loc_dist in ('clustered', 'uniform'):
        args = workload(2, Q, 8, D, 64, levels, P, dtype, loc_dist=loc_dist, seed=17)
        # many corners, not dense, the bins' entries within the float32 accumulator
        assert 2 * Q * 8 * L * P * 4 >= 1 << 18 and Q * L * P * 4 < 16 * N and Q * L * P * 8 <= N * D
        go = grad_out_for(args)
        say(f'  backward binned value gradient D={D} L={L} Q={Q} {dtype} {loc_dist} mask={with_mask}')
        grads, _ = gpu_grads(args, go, dtype, mask=mask)
        ref = gridsample.deform_attn_grads(*args, go.to(dtype), padding_mask=mask)
        for n in NAMES:
            check(f'binned D={D} {dtype} {loc_dist} d{n}', grads[n], ref[n], dtype)


@pytest.mark.parametrize('dtype,D', [(torch.float16, 32), (torch.bfloat16, 16), (torch.float32, 8)])
@pytest.mark.parametrize('with_mask', [False, True])
def test_self_attention_tile_gradients(dtype, D, with_mask):
    # as many queries as tokens: the bucketed scatter takes 8 x 4-pixel tiles of each level's map (query q at token
    # q), here on maps whose sides are not multiples of 8 or 4 (tiles cut at the right and bottom edges) and a map
    # narrower than a tile; encoder locations and uniform ones (every window then too large: the direct path)
    levels = [(25, 37), (13, 19), (7, 10), (3, 5)]
    N = sum(h * w for h, w in levels)
    mask = (torch.rand(1, N, generator=torch.Generator().manual_seed(4)) < 0.2) if with_mask else None
    for loc_dist in ('encoder', 'uniform'):
        for seed in range(31, 300):
            args = workload(1, N, 4, D, 64, levels, 4, dtype, loc_dist=loc_dist, seed=seed)
            if dtype != torch.float32 or boundary_distance(args[5], levels) >= 1e-5:
                break
        go = grad_out_for(args)
        say(f'  backward self-attention tiles N={N} D={D} {dtype} {loc_dist} mask={with_mask}')
        grads, _ = gpu_grads(args, go, dtype, mask=mask)
        ref = gridsample.deform_attn_grads(*args, go.to(dtype), padding_mask=mask)
        for n in NAMES:
            check(f'tiles D={D} {dtype} {loc_dist} d{n}', grads[n], ref[n], dtype)


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
@pytest.mark.parametrize('loc_dist', ['encoder', 'uniform'])
def test_dense_query_gradients_nine_levels(dtype, loc_dist):
    # the bucketed scatter finds the bounding boxes of 8 levels at a time: nine levels cross that boundary (a second
    # group of boxes, behind a barrier that waits for every wavefront to have read the first group's), with 2
    # points a level (18 samples a row, 28 rows a workgroup)
    levels = [(16, 16), (12, 12), (10, 10), (8, 8), (6, 6), (5, 5), (4, 4), (3, 3), (2, 2)]
    N = sum(h * w for h, w in levels)
    for Q in (2 * N, 2 * N - 3):
        args = workload(1, Q, 4, 16, 64, levels, 2, dtype, loc_dist=loc_dist, seed=21)
        go = grad_out_for(args)
        say(f'  backward dense queries, nine levels, Q={Q} {dtype} {loc_dist}')
        grads, _ = gpu_grads(args, go, dtype)
        ref = gridsample.deform_attn_grads(*args, go.to(dtype))
        for n in NAMES:
            check(f'nine levels Q={Q} {dtype} {loc_dist} d{n}', grads[n], ref[n], dtype)


@pytest.mark.parametrize('shape', ['rtdetr-b1', 'binned'])
def test_training_step_graph_replays_match_oracle(shape):
    # the training step (gradients set to None, forward, backward) captured in a graph, as the benchmark times it:
    # every replay must give all five gradients (the backward's accumulator is cleared by a kernel, not a memset),
    # each checked against the float64 oracle, with eager work on the device between the replays. 'binned': a decoder
    # shape of 2^18 corners and more, whose value gradient takes the binned kernels (their item counter is reset by
    # sort_count_kernel, their bin table computed from the device-resident shapes at every replay)
    if shape == 'rtdetr-b1':
        args = workload(1, 300, 8, 32, 256, RTDETR_LEVELS, 4, torch.float16, seed=11)
    else:
        args = workload(2, 400, 8, 32, 256, SORT_LEVELS['dino'], 4, torch.float16, loc_dist='clustered', seed=11)
    go = grad_out_for(args)
    ref = gridsample.deform_attn_grads(*args, go.to(torch.float16))
    dev = [None if t is None else t.cuda() for t in args]
    leaves = [t.requires_grad_(True) if (i in (0, 1, 2, 5, 6) and t is not None) else t for i, t in enumerate(dev)]
    g = go.to(torch.float16).cuda()

    def step():
        for t in leaves:
            if t is not None and t.requires_grad:
                t.grad = None
        torch.autograd.backward(td.ma_deform_attn_train(*leaves), g)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        for t in leaves:
            if t is not None and t.requires_grad:
                t.grad.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        say(f'  training step graph replay {i} ({shape})')
        grads = {n: None if leaves[j] is None else leaves[j].grad for n, j in zip(NAMES, (0, 1, 2, 5, 6))}
        for n in NAMES:
            check(f'replay {i} d{n}', grads[n], ref[n], torch.float16)
        with torch.no_grad():
            _ = dev[0].float().sum().item()  # eager work between replays


def test_module_training_step_matches_cpu():
    # MSDeformAttnLayer with grad: PyTorch prologue and output_proj, the library's operator; parameter gradients of
    # one step against the same module on the CPU in float64 (the reference path under autograd)
    torch.manual_seed(0)
    m = td.MSDeformAttnLayer(d_model=64, n_levels=2, n_heads=4, n_points=2)
    with torch.no_grad():  # non-trivial offsets and attention
        m.sampling_offsets.weight.normal_(0, 0.05)
        m.attention_weights.weight.normal_(0, 0.1)
    levels = [(12, 10), (6, 5)]
    shapes = torch.tensor(levels)
    sizes = shapes[:, 0] * shapes[:, 1]
    starts = torch.cat([sizes.new_zeros(1), sizes.cumsum(0)[:-1]])
    g = torch.Generator().manual_seed(3)
    hidden = torch.randn(2, 20, 64, generator=g)
    memory = torch.randn(2, int(sizes.sum()), 64, generator=g)
    ref_pts = torch.cat([torch.rand(2, 20, 1, 2, generator=g), torch.rand(2, 20, 1, 2, generator=g) * 0.3 + 0.05], -1)
    pos = torch.randn(2, 20, 64, generator=g) * 0.1

    def step(module, dev, dtype):
        module = module.to(dev, dtype)
        module.zero_grad()
        out, attn = module(hidden.to(dev, dtype), encoder_hidden_states=memory.to(dev, dtype),
                           position_embeddings=pos.to(dev, dtype), reference_points=ref_pts.to(dev, dtype),
                           spatial_shapes=shapes.to(dev), level_start_index=starts.to(dev))
        (out * out).sum().backward()
        return {n: p.grad.detach().double().cpu() for n, p in module.named_parameters()}

    import copy
    gpu = step(copy.deepcopy(m), 'cuda', torch.float32)
    cpu = step(copy.deepcopy(m), 'cpu', torch.float64)
    for n in cpu:
        scale = max(float(cpu[n].abs().max()), 1e-6)
        err = float((gpu[n] - cpu[n]).abs().max()) / scale
        assert err <= 5e-4, f'{n}: {err:.3g}'


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize('with_mask', [False, True])
def test_encoder_shape_gradients(dtype, with_mask):
    # self-attention shapes (every token a query, sampling around itself, as encoder layers call the operator):
    # neighbouring queries add into the same value-gradient rows many times over. Q = N = 4080 on four levels, and
    # Q = 4077; a padding mask drops tokens as in the other paths
    levels = [(48, 64), (24, 32), (12, 16), (6, 8)]
    for Q in (4080, 4077):
        args = workload(1, Q, 8, 32, 64, levels, 4, dtype, loc_dist='encoder', seed=5)
        N = args[0].shape[1]
        mask = (torch.rand(1, N, generator=torch.Generator().manual_seed(6)) < 0.2) if with_mask else None
        go = grad_out_for(args)
        say(f'  backward encoder shape Q={Q} {dtype} mask={with_mask}')
        grads, _ = gpu_grads(args, go, dtype, mask=mask)
        ref = gridsample.deform_attn_grads(*args, go.to(dtype), padding_mask=mask)
        for n in NAMES:
            check(f'encoder Q={Q} {dtype} d{n}', grads[n], ref[n], dtype)



@pytest.mark.parametrize('dtype,D,nlev', [(torch.float16, 8, 2), (torch.bfloat16, 16, 2), (torch.float16, 64, 2),
                                          (torch.float32, 4, 2), (torch.float32, 32, 2), (torch.float32, 64, 3)])
@pytest.mark.parametrize('loc_dist', ['encoder', 'uniform'])
def test_dense_query_gradients(dtype, D, nlev, loc_dist):
    # many queries per token (Q = 2N, 4 points a level: 16 or more corner hits per token and head on average), so the
    # value gradient goes through the bucketed scatter (scatter_bucket_kernel) and the location and weight gradients
    # through loc_attn_backward_kernel: with encoder locations each level's corners of consecutive queries fit its
    # window and are summed per pixel; with uniform ones they do not and the kernel adds them directly. Head widths 4
    # to 64 in every 16/32-bit type (1 to 16 lanes a corner row in the dot products), two levels (8 samples a row) or
    # three (12: 21 rows a workgroup, four threads idle), Q = 2N and 2N - 2 (a ragged last tile)
    levels = [(24, 32), (12, 16), (6, 8)][:nlev]
    N = sum(h * w for h, w in levels)
    for Q in (2 * N, 2 * N - 2):
        # the location gradient of bilinear sampling jumps where a sample crosses a pixel boundary; a sample within
        # float32 rounding of one (x = loc * W - 0.5 carries about 2e-6 pixel of rounding at W = 32) is floored to
        # one side here and possibly the other in the float64 oracle, so the seed is the first from 7 whose samples
        # all lie at least 1e-5 pixel from a boundary
        for seed in range(7, 200):
            args = workload(1, Q, 4, D, 64, levels, 4, dtype, loc_dist=loc_dist, seed=seed)
            if boundary_distance(args[5], levels) >= 1e-5:
                break
        assert boundary_distance(args[5], levels) >= 1e-5
        go = grad_out_for(args)
        say(f'  backward dense queries Q={Q} D={D} L={nlev} {dtype} {loc_dist}')
        grads, _ = gpu_grads(args, go, dtype)
        ref = gridsample.deform_attn_grads(*args, go.to(dtype))
        for n in NAMES:
            check(f'dense Q={Q} D={D} {dtype} {loc_dist} d{n}', grads[n], ref[n], dtype)
