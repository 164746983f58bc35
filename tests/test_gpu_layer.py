"""The decoder-layer entries on the GPU against the float64 layer oracle (oracle/layer.py, itself pinned against
HF transformers' RTDetrMultiscaleDeformableAttention in tests/test_layer.py).

Tolerances: the output as the operator's tests (float32 atol 2e-5 / rtol 1e-4 scaled by max|ref|; float16 and
bfloat16 2e-2 of max|ref| as relative error, and elementwise atol 3e-3 / 2e-2 + rtol); the attention weights and
locations, computed in float32 from the same inputs, within 2e-5 (float32, float16) / 1e-4 (bfloat16, whose
query split into two halves keeps 16 significant bits) of the oracle's.
"""

import numpy as np
import pytest
import torch

import marearts_tinydeform_amd as td
from marearts_tinydeform_amd import _native
from oracle import layer as olayer
from inputs import LAYER_CASES, RTDETR_LEVELS, make_layer, to

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (2e-5, 1e-4), torch.float16: (3e-3, 3e-3), torch.bfloat16: (2e-2, 2e-2),
       torch.float64: (1e-10, 1e-10)}
REL = {torch.float32: 1e-4, torch.float16: 2e-2, torch.bfloat16: 2e-2, torch.float64: 1e-10}
LOC_TOL = {torch.float32: 2e-5, torch.float16: 2e-5, torch.bfloat16: 1e-4, torch.float64: 1e-12}


def say(msg):
    print(msg, flush=True)


def check(name, got, ref, dtype):
    got = got.double().cpu().numpy()
    assert got.shape == ref.shape, f'{name}: shape {got.shape} != {ref.shape}'
    atol, rtol = TOL[dtype]
    scale = max(float(np.abs(ref).max()), 1.0) if ref.size else 1.0
    err = np.abs(got - ref)
    bad = err > atol * scale + rtol * np.abs(ref)
    assert not bad.any(), f'{name}: {int(bad.sum())} out of tolerance, max |diff| {err.max():.3g}'
    if ref.size:
        assert err.max() / scale <= REL[dtype], f'{name}: relative error {err.max() / scale:.3g}'


def run_layer(dev, mode, mask=None, want_attn=True):
    with torch.inference_mode():
        res = td.ma_deform_attn_layer(*dev[:15], position_embeddings=dev[15], padding_mask=mask, mode=mode,
                                      return_attention_weights=want_attn)
    torch.cuda.synchronize()
    return res


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize('case', LAYER_CASES, ids=[c[0] for c in LAYER_CASES])
def test_layer_cases(case, dtype):
    name, B, Q, H, D, C, levels, P, rd, rl = case
    a = make_layer(B, Q, H, D, C, levels, P, rd, rl, dtype=dtype)
    ref, ref_attn = olayer.layer(*a[:15], position_embeddings=a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    for mode in ('fused', 'project', 'auto'):
        say(f'  {name} {dtype} [{mode}]')
        out, attn = run_layer(dev, mode)
        check(f'{name} {dtype} [{mode}]', out, ref, dtype)
        np.testing.assert_allclose(attn.double().cpu().numpy(), ref_attn, rtol=0,
                                   atol=max(LOC_TOL[dtype], 2 ** -8 if dtype == torch.bfloat16 else
                                            2 ** -11 if dtype == torch.float16 else 0))


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
def test_locations_in_float32(dtype):
    """loc / attn as the kernels compute them (float32, before any rounding), fused and standalone prologue."""
    a = make_layer(2, 45, 8, 32, 256, RTDETR_LEVELS, 4, 4, '1', dtype=dtype)
    ref_loc, ref_attn = olayer.locations(a[0], a[2], a[3], a[5], a[6], a[7], a[8], a[13], a[14], a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    hidden, memory, rp, shapes, starts, ow, ob, aw, ab, vw, vb = dev[:11]
    with torch.inference_mode():
        loc, attn = _native.layer_prologue(hidden, dev[15], rp, ow, ob, aw, ab, shapes, 8, 4)
        _, (floc, fattn) = _native.layer_fused_forward(hidden, dev[15], rp, ow, ob, aw, ab, memory, vw, vb, shapes,
                                                       starts, 8, 4, return_locations=True)
    torch.cuda.synchronize()
    tol = LOC_TOL[dtype]
    for nm, l_, a_ in (('prologue', loc, attn), ('fused', floc, fattn)):
        say(f'  locations {dtype} [{nm}]')
        assert l_.dtype == torch.float32 and a_.dtype == torch.float32
        np.testing.assert_allclose(l_.double().cpu().numpy(), ref_loc, rtol=0, atol=tol)
        np.testing.assert_allclose(a_.double().cpu().numpy(), ref_attn, rtol=0, atol=tol)


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
def test_large_prologue_takes_the_gemm_route(dtype):
    # >= 8e8 multiply-adds in the query projections: project mode runs them on the GEMM (hidden . W^T + pos . W^T in
    # float32) and finalizes softmax and locations in place; boxes with 64 samples per head (one row per wavefront)
    # and points per level with 12 (four rows per wavefront), with and without bias. In 16 bits both projections
    # share one launch of 64 x 128 tiles: 600 and 1800 rows end in a partial row block, 2 * 192 and 192 columns in
    # a partial column block, and without position embeddings the tiles take one operand.
    for name, (B, Q, H, D, C, levels, P, rd, rl, bias, pos) in {
            'boxes': (2, 300, 16, 32, 512, [(40, 40), (20, 20), (10, 10), (5, 5)], 16, 4, '1', True, True),
            'points per level': (2, 900, 16, 32, 1024, [(48, 40), (24, 20), (12, 10)], 4, 2, 'L', False, True),
            'no position': (1, 700, 16, 32, 1024, [(40, 40), (20, 20), (10, 10), (5, 5)], 8, 4, '1', True,
                            False)}.items():
        a = make_layer(B, Q, H, D, C, levels, P, rd, rl, dtype=dtype, bias=bias, pos=pos)
        ref, ref_attn = olayer.layer(*a[:15], position_embeddings=a[15])
        ref_loc, _ = olayer.locations(a[0], a[2], a[3], a[5], a[6], a[7], a[8], H, P, position_embeddings=a[15])
        dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
        say(f'  gemm route {name} {dtype}')
        loc, attn = _native.layer_prologue(dev[0], dev[15], dev[2], dev[5], dev[6], dev[7], dev[8], dev[3], H, P)
        torch.cuda.synchronize()
        lt = LOC_TOL[dtype]
        assert np.abs(loc.double().cpu().numpy() - ref_loc).max() <= lt, f'{name}: locations'
        assert np.abs(attn.double().cpu().numpy() - ref_attn).max() <= lt, f'{name}: attention weights'
        out, got_attn = run_layer(dev, 'project')
        check(f'{name} {dtype} [project]', out, ref, dtype)
        # fused mode takes the same prologue, then the fused kernel on its float32 locations
        say(f'  gemm route {name} {dtype} [fused]')
        out, got_attn = run_layer(dev, 'fused')
        check(f'{name} {dtype} [fused]', out, ref, dtype)
        np.testing.assert_allclose(got_attn.double().cpu().numpy(), ref_attn, rtol=0, atol=max(lt, 2e-2))
        # through the C ABI, without location buffers the fused entry asks for them, launching nothing
        hidden, memory, rp, shapes, starts, ow, ob, aw, ab, vw, vb = dev[:11]
        N, Cq = memory.shape[1], hidden.shape[2]
        out = torch.empty(B, Q, H * D, dtype=dtype, device='cuda')
        args = [_native.DTYPE_CODES[dtype], hidden.data_ptr(), _native._ptr(dev[15]), rp.data_ptr(), rp.shape[2],
                rp.shape[3], ow.data_ptr(), _native._ptr(ob), aw.data_ptr(), _native._ptr(ab), memory.data_ptr(),
                vw.data_ptr(), _native._ptr(vb), shapes.data_ptr(), starts.data_ptr(), None, out.data_ptr()]
        sizes = [B, Q, N, Cq, C, H, D, len(levels), P, None]
        assert _native.lib.td_layer_fused_forward(*args, None, None, *sizes) == _native.TD_E_WORKSPACE


@pytest.mark.parametrize('Q,in_kernel', [(200, False), (50, True)])
def test_wide_projection_weights(Q, in_kernel):
    # 8 heads x 4 levels x 16 points over C = 512: 196 KB of projection weights per head, under the GEMM route's
    # 8e8 multiply-adds. From 200 query rows the fused layer runs the standalone prologue and then the fused kernel
    # (and through the C ABI asks for location buffers); with 50 it keeps the prologue inside the fused kernel.
    dtype = torch.bfloat16
    B, H, D, C, levels, P = 1, 8, 64, 512, [(40, 40), (20, 20), (10, 10), (5, 5)], 16
    a = make_layer(B, Q, H, D, C, levels, P, 4, '1', dtype=dtype)
    ref, ref_attn = olayer.layer(*a[:15], position_embeddings=a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    say(f'  wide weights Q{Q} [fused]')
    out, got_attn = run_layer(dev, 'fused')
    check(f'wide weights Q{Q} [fused]', out, ref, dtype)
    hidden, memory, rp, shapes, starts, ow, ob, aw, ab, vw, vb = dev[:11]
    out = torch.empty(B, Q, H * D, dtype=dtype, device='cuda')
    args = [_native.DTYPE_CODES[dtype], hidden.data_ptr(), dev[15].data_ptr(), rp.data_ptr(), rp.shape[2], rp.shape[3],
            ow.data_ptr(), ob.data_ptr(), aw.data_ptr(), ab.data_ptr(), memory.data_ptr(), vw.data_ptr(),
            vb.data_ptr(), shapes.data_ptr(), starts.data_ptr(), None, out.data_ptr(), None, None,
            B, Q, memory.shape[1], hidden.shape[2], C, H, D, len(levels), P, None]
    rc = _native.lib.td_layer_fused_forward(*args)
    torch.cuda.synchronize()
    if in_kernel:
        assert rc == 0  # the core, before output_proj: apply it in float64 to compare with the layer
        o_w, o_b = dev[11].double(), dev[12].double()
        check(f'wide weights Q{Q} [C ABI]', out.double() @ o_w.T + o_b, ref, dtype)
    else:
        assert rc == _native.TD_E_WORKSPACE


@pytest.mark.parametrize('L,P,dtype,ref_dim,ref_levels', [
    (1, 4, torch.bfloat16, 4, '1'), (2, 4, torch.float16, 4, '1'), (4, 4, torch.bfloat16, 4, '1'),
    (4, 8, torch.float16, 4, '1'),
    # point references (divided by each level's width and height), one per level, and boxes per level
    (4, 4, torch.bfloat16, 2, 'L'), (2, 8, torch.float16, 2, 'L'), (2, 2, torch.float16, 2, '1'),
    (4, 2, torch.bfloat16, 4, 'L')])
def test_gemm_route_finalizes_in_its_epilogue(L, P, dtype, ref_dim, ref_levels):
    # In 16 bits with L * P a power of two from 4 to 64 the projections' epilogue turns offsets into locations and
    # logits into softmax weights (a head's L * P logits of a row sit in one to four lanes of one or two 16-column
    # blocks); the other cases of the GEMM route (64 samples, 12 samples) are in test_large_prologue_takes_the_gemm_route.
    # Enough rows for the route (8e8 multiply-adds at 16 heads over 1024 channels), ending in a partial row block.
    H, Cq, LP = 16, 1024, L * P
    rows = -(-int(8e8) // (H * 3 * LP * Cq))
    B, Q = 2, rows // 2 + 7
    levels = [(8, 10), (4, 5), (2, 3), (1, 2)][:L]
    a = make_layer(B, Q, H, 32, Cq, levels, P, ref_dim, ref_levels, dtype=dtype)
    ref_loc, ref_attn = olayer.locations(a[0], a[2], a[3], a[5], a[6], a[7], a[8], H, P, position_embeddings=a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    say(f'  epilogue finalize L{L} P{P} {dtype} ref {ref_dim}/{ref_levels} B{B} Q{Q}')
    loc, attn = _native.layer_prologue(dev[0], dev[15], dev[2], dev[5], dev[6], dev[7], dev[8], dev[3], H, P)
    torch.cuda.synchronize()
    lt = LOC_TOL[dtype]
    assert np.abs(loc.double().cpu().numpy() - ref_loc).max() <= lt, 'locations'
    assert np.abs(attn.double().cpu().numpy() - ref_attn).max() <= lt, 'attention weights'


def test_float64_layer_takes_the_standalone_prologue():
    a = make_layer(2, 21, 4, 16, 64, [(12, 18), (6, 9)], 4, 2, 'L', dtype=torch.float64)
    ref, ref_attn = olayer.layer(*a[:15], position_embeddings=a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    for mode in ('fused', 'project'):
        say(f'  float64 [{mode}]')
        out, attn = run_layer(dev, mode)
        check(f'float64 [{mode}]', out, ref, torch.float64)
        np.testing.assert_allclose(attn.cpu().numpy(), ref_attn, rtol=0, atol=1e-12)
    # without location buffers the fused entry reports that it needs them, launching nothing
    lib = _native.lib
    hidden, memory, rp, shapes, starts, ow, ob, aw, ab, vw, vb = dev[:11]
    out = torch.empty(2, 21, 64, dtype=torch.float64, device='cuda')
    rc = lib.td_layer_fused_forward(3, hidden.data_ptr(), None, rp.data_ptr(), 2, 2, ow.data_ptr(), ob.data_ptr(),
                                    aw.data_ptr(), ab.data_ptr(), memory.data_ptr(), vw.data_ptr(), vb.data_ptr(),
                                    shapes.data_ptr(), starts.data_ptr(), None, out.data_ptr(), None, None,
                                    2, 21, memory.shape[1], 64, 64, 4, 16, 2, 4, None)
    assert rc == _native.TD_E_WORKSPACE


@pytest.mark.parametrize('dtype', [torch.float16, torch.bfloat16])
def test_layer_padding_mask_and_no_bias(dtype):
    a = make_layer(2, 60, 8, 32, 256, [(40, 40), (20, 20), (10, 10)], 4, 2, 'L', dtype=dtype, bias=False, pos=False)
    N = a[1].shape[1]
    mask = torch.zeros(2, N, dtype=torch.bool)
    mask[1, :] = torch.rand(N, generator=torch.Generator().manual_seed(5)) < 0.4  # image 1 partly padded
    ref, _ = olayer.layer(*a[:15], position_embeddings=None, padding_mask=mask)
    dev = to(a[:13], 'cuda') + a[13:15] + [None]
    for mode in ('fused', 'project'):
        say(f'  mask {dtype} [{mode}]')
        out = run_layer(dev, mode, mask=mask.cuda(), want_attn=False)
        check(f'mask {dtype} [{mode}]', out, ref, dtype)


def test_layer_without_output_projection():
    a = make_layer(1, 40, 8, 32, 256, RTDETR_LEVELS, 4, 4, '1', dtype=torch.float16, out_proj=False)
    ref, _ = olayer.layer(*a[:15], position_embeddings=a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    out = run_layer(dev, 'fused', want_attn=False)
    assert out.shape == (1, 40, 256)
    check('no output_proj', out, ref, torch.float16)


def test_module_on_gpu_matches_cpu():
    torch.manual_seed(0)
    m = td.MSDeformAttnLayer(d_model=256, n_levels=3, n_heads=8, n_points=4)
    with torch.no_grad():  # offsets and attention that depend on the query
        m.sampling_offsets.weight.normal_(0, 0.05)
        m.attention_weights.weight.normal_(0, 0.05)
    a = make_layer(2, 50, 8, 32, 256, RTDETR_LEVELS, 4, 4, '1', dtype=torch.float32)
    hidden, memory, ref, shapes, starts = a[:5]
    kw = dict(hidden_states=hidden, encoder_hidden_states=memory, position_embeddings=a[15], reference_points=ref,
              spatial_shapes=shapes, level_start_index=starts)
    with torch.no_grad():
        want, want_attn = m(**kw)
        mg = m.cuda()
        got, got_attn = mg(**{k: v.cuda() for k, v in kw.items()})
    torch.cuda.synchronize()
    scale = float(want.abs().max())
    assert float((got.cpu() - want).abs().max()) <= 1e-4 * scale
    assert float((got_attn.cpu() - want_attn).abs().max()) <= 2e-5


def test_layer_graph_capture_replays_match_eager():
    a = make_layer(1, 300, 8, 32, 256, RTDETR_LEVELS, 4, 4, '1', dtype=torch.float16)
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    with torch.inference_mode():
        eager = run_layer(dev, 'fused', want_attn=False).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            run_layer(dev, 'fused', want_attn=False)
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_out = td.ma_deform_attn_layer(*dev[:15], position_embeddings=dev[15], mode='fused')
        for i in range(3):
            static_out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(static_out, eager), f'replay {i}'


@pytest.mark.parametrize('dtype', [torch.float32, torch.float16, torch.bfloat16])
def test_encoder_layer_self_attention(dtype):
    """The layer as a Deformable-DETR / DINO encoder calls it: the queries are the memory tokens (hidden states =
    memory, Q = N), the reference points are every token's centre, repeated per level ([B, N, L, 2]), and each
    query samples a few pixels around itself; all three modes against the oracle."""
    from inputs import token_centres
    levels = [(32, 48), (16, 24), (8, 12)]
    a = make_layer(2, 1, 8, 32, 256, levels, 4, 2, 'L', dtype=torch.float32)
    memory = a[1]
    B, N = memory.shape[:2]
    ref = token_centres(levels)[None, :, None, :].expand(B, N, len(levels), 2).contiguous()
    a = [t.to(dtype) if isinstance(t, torch.Tensor) and t.is_floating_point() else t for t in a]
    a[0], a[2] = memory.to(dtype), ref.to(dtype)  # hidden states = memory; token-centre reference points
    a[15] = (torch.randn(B, N, memory.shape[2], generator=torch.Generator().manual_seed(4)) * 0.5).to(dtype)
    ref_out, ref_attn = olayer.layer(*a[:15], position_embeddings=a[15])
    dev = to(a[:13], 'cuda') + a[13:15] + to(a[15:], 'cuda')
    for mode in ('fused', 'project', 'auto'):
        say(f'  encoder layer {dtype} [{mode}] N={N}')
        out, attn = run_layer(dev, mode)
        check(f'encoder layer {dtype} [{mode}]', out, ref_out, dtype)
