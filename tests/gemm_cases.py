"""Shapes of the value-projection parity tests (tests/test_gpu_parity.py), each with the kernel the size rule
(td_value_proj_plan) must pick for it. tests/test_gemm_plan.py checks on the CPU that the tags hold and that every
kernel the rule can pick for any shape has at least one of these cases; the GPU tests run them against the oracle.

Kernel numbers (csrc/td_gemm.hip): 0 generic VALU; 2, 5, 23, 24, 25 A-in-registers MFMA tiles; 9, 13 both operands
through LDS; 14 direct-to-LDS 256 x 128 tiles, one per workgroup; 18 persistent direct-to-LDS 256 x 256 tiles (one
workgroup per CU walking its tiles; last tiles moved back to end at M and NO); 22 the streaming kernel (W resident in
registers, tokens streamed through LDS).
"""

import torch

F16, BF16, F32, F64 = torch.float16, torch.bfloat16, torch.float32, torch.float64

# (B, N, C, HD) run in every dtype, every row checked: {dtype: kernel} for each shape
SMALL = [
    ((1, 8400, 256, 256), {F16: 25, BF16: 25, F32: 25, F64: 0}),
    ((4, 9000, 256, 256), {F16: 22, BF16: 22, F32: 5, F64: 0}),
    ((2, 8192, 128, 1024), {F16: 13, BF16: 13, F32: 2, F64: 0}),
    ((2, 77, 40, 48), {F16: 24, BF16: 24, F32: 24, F64: 0}),
    ((1, 130, 96, 72), {F16: 24, BF16: 24, F32: 24, F64: 0}),
    ((3, 5, 8, 16), {F16: 24, BF16: 24, F32: 24, F64: 0}),
    ((1, 33, 1024, 64), {F16: 24, BF16: 24, F32: 25, F64: 0}),
    ((1, 1200, 256, 256), {F16: 24, BF16: 24, F32: 23, F64: 0}),
]

# 16-bit (M, K, NO, kernel), deep K; rows checked on a sample that includes the first and the last (partial) M tile
DEEP_K = [
    (1037, 512, 200, 23),
    (5000, 576, 136, 25),
    (300, 1024, 1024, 23),     # the decoder layer's output projection at C = 1024, 300 queries
    (3600, 1024, 1024, 9),     # both operands through LDS, K chunks of 128
    (21760, 1024, 1024, 18),   # C = 1024 limit shape at batch 1: persistent 256 x 256 tiles, about 1.3 per workgroup
    (21760, 512, 512, 18),     # a C = 512 model at batch 1
    (43557, 1024, 1008, 18),   # M and NO off the tile sizes: the last token and channel tiles moved back, overlapping
    (43557, 1024, 1000, 14),   # NO not a multiple of 16: the 256 x 128 tiles
    (30001, 768, 768, 18),     # three channel tiles: 30 workgroups per XCD, each keeping its channel tile
    (60000, 512, 320, 18),     # two channel tiles overlapping by 192 channels, two tiles per workgroup
    (131072, 512, 512, 18),    # four tiles per workgroup
    (12000, 1024, 1024, 18),   # 188 tiles: fewer workgroups than CUs, one tile each
    (9000, 520, 256, 9),       # K >= 512 but not a multiple of 64
    (8400, 512, 256, 14),      # direct-to-LDS from 8000 rows even on a small grid (66 tiles of 256 x 128)
    (6000, 1024, 1024, 14),    # more than one round of 128 x 128 tiles
]

# 16-bit (M, K, bias, kernel) with NO = 256, every row checked: the streaming kernel from 14000 rows at K = 256 and
# 8000 at K = 128. Each CU takes an equal share of M (shares differ by one row) in steps of 32 tokens, the last one
# partial: one step per CU (8000, 8100 at K = 128, where fewer than 256 workgroups run), two (16384), shares off the
# step size (14000, 36001, 44447, 20011, 70003, 76801, 100003), whole steps (131072 = 256 x 16 x 32), with and
# without bias, up to 22 steps per CU (177784 at K = 128).
STREAM = [
    (14000, 256, True, 22), (16384, 256, True, 22), (16800, 256, False, 22), (33600, 256, False, 22),
    (36001, 256, True, 22), (44447, 256, False, 22), (67200, 256, True, 22), (76801, 256, False, 22),
    (88892, 256, True, 22), (131072, 256, True, 22), (8000, 128, True, 22), (8100, 128, False, 22),
    (20011, 128, True, 22), (44447, 128, False, 22), (70003, 128, True, 22), (100003, 128, True, 22),
    (177784, 128, False, 22),
    (13999, 256, True, 25),    # one row short of the streaming kernel's range
    (7999, 128, True, 25),
]

# 16-bit (M, K, NO, kernel): a bias view 2 bytes off a 16-byte boundary. The streaming kernel reads the bias with
# 16-byte loads, so such a bias must fall back to the tiled kernels.
BIAS_OFFSET = [
    (16800, 256, 256, 25),
    (67200, 256, 256, 13),
    (21760, 1024, 1024, 14),   # the persistent tiles read the bias with 16-byte loads too
]

# (M, K, NO, offsets, kernel) in float32, float16 and bfloat16: memory 4 bytes off a 16-byte boundary, or K not a
# multiple of 16 bytes: the generic VALU kernel
UNALIGNED = [
    (1000, 256, 256, {'memory': 4}, 0),
    (333, 38, 72, None, 0),
]

# head-major outputs (B, N, C, H, D) per dtype: {shape: kernel}
HEADS = {
    F16: [((1, 8400, 256, 8, 32), 25), ((4, 9000, 256, 8, 32), 22), ((2, 8192, 128, 32, 32), 13),
          ((3, 77, 40, 6, 8), 24), ((2, 2501, 576, 17, 8), 25), ((2, 30001, 256, 8, 32), 22),
          ((3, 20011, 128, 16, 16), 22), ((4, 8400, 256, 8, 32), 22), ((1, 21760, 1024, 32, 32), 18),
          ((2, 21760, 512, 32, 16), 18), ((1, 21760, 1024, 128, 8), 14)],
    BF16: [((1, 8400, 256, 8, 32), 25), ((2, 30001, 256, 8, 32), 22), ((5, 131, 96, 3, 24), 24),
           ((8, 8400, 256, 8, 32), 22), ((1, 3600, 1024, 32, 32), 9)],
    F32: [((1, 8400, 256, 8, 16), 25), ((2, 77, 40, 5, 4), 24), ((3, 1000, 64, 2, 12), 23)],
    F64: [((2, 77, 40, 4, 2), 0), ((1, 300, 256, 8, 8), 0)],
}


def all_cases():
    """Every (dtype, M, K, NO, bias, offsets, heads, N, kernel) of the lists above."""
    out = []
    for (B, N, C, HD), kern in SMALL:
        for dt, k in kern.items():
            out.append((dt, B * N, C, HD, True, None, None, None, k))
    for dt in (F16, BF16):
        for M, K, NO, k in DEEP_K:
            out.append((dt, M, K, NO, True, None, None, None, k))
        for M, K, bias, k in STREAM:
            out.append((dt, M, K, 256, bias, None, None, None, k))
    for M, K, NO, k in BIAS_OFFSET:
        out.append((F16, M, K, NO, True, {'bias': 2}, None, None, k))
    for dt in (F32, F16, BF16):
        for M, K, NO, offsets, k in UNALIGNED:
            out.append((dt, M, K, NO, True, offsets, None, None, k))
    for dt, cases in HEADS.items():
        for (B, N, C, H, D), k in cases:
            out.append((dt, B * N, C, H * D, True, None, H, N, k))
    return out
