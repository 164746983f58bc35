"""The value projection's size rule, evaluated on the CPU through td_value_proj_plan (no kernel is launched).

Every case of tests/gemm_cases.py must get the kernel it is tagged with, and every kernel the rule can pick for any
shape (a sweep over M, K and NO in every dtype, plus the alignment cases) must be one that some GPU parity case runs.
"""

import itertools

import pytest

from marearts_tinydeform_amd import _native
from gemm_cases import BF16, F16, F32, F64, all_cases

pytestmark = pytest.mark.skipif(_native.lib is None, reason='libtinydeform.so is not built')


def test_every_parity_case_gets_its_kernel():
    for dt, M, K, NO, bias, offsets, heads, N, kern in all_cases():
        got = _native.value_proj_plan(dt, M, K, NO, bias=bias, offsets=offsets, heads=heads, N=N)
        assert got == kern, f'{dt} M={M} K={K} NO={NO} bias={bias} offsets={offsets} heads={heads}: kernel {got}, ' \
                            f'tagged {kern}'


def covered():
    cov = {}
    for dt, *_, kern in all_cases():
        cov.setdefault(dt, set()).add(kern)
    return cov


def test_every_reachable_kernel_has_a_parity_case():
    cov = covered()
    Ms = sorted({int(1.37 ** i) for i in range(40)} | {300, 600, 3600, 7999, 8000, 8400, 13999, 14000, 21760, 43520, 67200,
                                                       88892, 177784, 300000})
    Ks = (8, 40, 64, 96, 128, 256, 512, 520, 576, 1024, 2048)
    NOs = (16, 48, 64, 136, 200, 256, 512, 1000, 1024, 2048)
    reach = {}
    for dt in (F16, BF16, F32, F64):
        for M, K, NO in itertools.product(Ms, Ks, NOs):
            for bias, offsets in ((True, None), (False, None), (True, {'bias': 2}), (True, {'memory': 2}),
                                  (True, {'weight': 4})):
                reach.setdefault(dt, set()).add(_native.value_proj_plan(dt, M, K, NO, bias=bias, offsets=offsets))
            if NO % 8 == 0 and K % 8 == 0:
                D = 32 if NO % 32 == 0 else 8
                reach[dt].add(_native.value_proj_plan(dt, M, K, NO, heads=NO // D, N=M))
    for dt in reach:
        missing = reach[dt] - cov.get(dt, set())
        assert not missing, f'{dt}: kernels {sorted(missing)} are reachable but no GPU parity case runs them'
    # the sweep reaches every kernel of the rule (a guard against the sweep itself going stale)
    assert reach[F16] == reach[BF16] == {0, 9, 13, 14, 18, 22, 23, 24, 25}
    assert reach[F32] == {0, 2, 5, 23, 24, 25}
    assert reach[F64] == {0}


def test_streaming_kernel_needs_an_aligned_bias():
    # the streaming kernel reads the bias with 16-byte loads: any bias offset leaves it
    assert _native.value_proj_plan(F16, 67200, 256, 256) == 22
    assert _native.value_proj_plan(F16, 67200, 256, 256, bias=False) == 22
    for off in (2, 4, 8):
        assert _native.value_proj_plan(F16, 67200, 256, 256, offsets={'bias': off}) != 22
    assert _native.value_proj_plan(F16, 67200, 256, 256, offsets={'bias': 16}) == 22
    # so must memory, weight and value
    for k in ('memory', 'weight', 'value'):
        assert _native.value_proj_plan(BF16, 67200, 256, 256, offsets={k: 8}) != 22


def test_persistent_tiles_need_their_alignments():
    # the persistent 256 x 256 tiles store 16 channels per lane as two 16-byte vectors and read the bias the same way
    assert _native.value_proj_plan(F16, 43520, 1024, 1024) == 18
    assert _native.value_proj_plan(F16, 43520, 1024, 1024, bias=False) == 18
    for k in ('bias', 'value'):
        assert _native.value_proj_plan(BF16, 43520, 1024, 1024, offsets={k: 8}) == 14
    assert _native.value_proj_plan(F16, 43520, 1024, 1000) == 14          # NO % 16 != 0
    assert _native.value_proj_plan(F16, 43520, 1024, 1024, heads=128, N=43520) == 14  # D = 8
    assert _native.value_proj_plan(F16, 43520, 1024, 1024, heads=64, N=43520) == 18   # D = 16
    assert _native.value_proj_plan(F16, 8400, 512, 512) == 14             # 66 tiles of 256 x 256


def test_plan_rejects_bad_sizes():
    with pytest.raises(RuntimeError):
        _native.value_proj_plan(F16, -1, 256, 256)
    with pytest.raises(RuntimeError):
        _native.value_proj_plan(F16, 100, 256, 256, heads=3, N=100)


def test_bench_names_the_kernel_the_rule_picks():
    # bench.py attributes measured time and traffic to the value GEMM's kernel by name (gemm_kernel); it must name
    # the family td_value_proj_plan picks, for aligned row-major problems with a bias
    import bench
    family = {0: 'gemm_generic_kernel', 2: 'gemm_mfma_kernel', 5: 'gemm_mfma_kernel', 23: 'gemm_mfma_kernel',
              24: 'gemm_mfma_kernel', 25: 'gemm_mfma_kernel', 9: 'gemm_lds_kernel', 13: 'gemm_lds_kernel',
              14: 'gemm_dma_kernel', 18: 'gemm_dma_persistent_kernel', 22: 'gemm_stream_kernel'}
    Ms = (300, 2400, 7999, 8000, 8400, 14000, 21760, 30001, 43520, 67200, 177784)
    for dt, s in ((F16, 2), (BF16, 2)):
        for M, K, NO in itertools.product(Ms, (128, 256, 512, 768, 1024), (256, 320, 512, 768, 1000, 1024)):
            got = bench.gemm_kernel(M, K, NO, s)
            want = family[_native.value_proj_plan(dt, M, K, NO)]
            assert got == want, f'M={M} K={K} NO={NO}: bench names {got}, the rule picks {want}'
