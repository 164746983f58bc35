// Shared by the value-projection GEMM kernels (td_gemm.hip, td_gemm_dma.hip): launch parameters, the XCD-aware tile
// numbering and the 16-byte K block of an MFMA.
#pragma once

#include "td_internal.h"

namespace td {

struct GemmParams {
    const void* a;
    const void* w;
    const void* bias;
    void* c;
    int M, K, NO;
    int mt, nt;  // tile counts
    int per_xcd;
    const void* a2 = nullptr;  // second A operand of the two-operand form (C = A . W^T + A2 . W^T + bias)
    // head-major output (hm_D > 0): row m = b * hm_N + t and column n = h * hm_D + d go to
    // C[((b * H + h) * hm_N + t) * hm_D + d] with H = NO / hm_D, i.e. C is [B, H, N, D]; hm_D is a multiple of the
    // 16-byte vector
    int hm_N = 0, hm_D = 0;
    FastDiv hm_ndiv, hm_ddiv;  // division by hm_N and hm_D
};

// Element offset of output (m, n) = out_row(m) + out_col(n): row-major [M, NO], or head-major (GemmParams::hm_D)
__device__ __forceinline__ size_t out_row(const GemmParams& p, int m) {
    if (p.hm_D == 0) return static_cast<size_t>(m) * p.NO;
    const int b = static_cast<int>(fast_div(p.hm_ndiv, static_cast<uint32_t>(m))), t = m - b * p.hm_N;
    return static_cast<size_t>(b) * p.hm_N * p.NO + static_cast<size_t>(t) * p.hm_D;
}
__device__ __forceinline__ size_t out_col(const GemmParams& p, int n) {
    if (p.hm_D == 0) return static_cast<size_t>(n);
    const int h = static_cast<int>(fast_div(p.hm_ddiv, static_cast<uint32_t>(n))), d = n - h * p.hm_D;
    return static_cast<size_t>(h) * p.hm_N * p.hm_D + d;
}
__device__ __forceinline__ size_t out_index(const GemmParams& p, int m, int n) { return out_row(p, m) + out_col(p, n); }

// Linear tile index for this workgroup; -1 when the workgroup has no tile. Workgroups are dealt to the 8 XCDs
// round-robin, so consecutive tiles (the N tiles of one M tile) land on one XCD and share its L2.
__device__ __forceinline__ int tile_of(const GemmParams& p, int id) {
    const int tile = (id % kXcds) * p.per_xcd + id / kXcds;
    return tile < p.mt * p.nt ? tile : -1;
}
__device__ __forceinline__ int tile_of(const GemmParams& p) { return tile_of(p, static_cast<int>(blockIdx.x)); }

// One 16-byte K block of an MFMA: 16-bit types take one v_mfma_f32_16x16x32 (K = 32 = 4 lane groups x 8),
// float32 takes four v_mfma_f32_16x16x4_f32 on the components of a float4 (K = 16 = 4 lane groups x 4, lane group
// g holding k = 4g..4g+3; A and B use the same k order, so the sum covers each k once).
template <typename T>
struct KBlock;
template <>
struct KBlock<f16> {
    static constexpr int kK = 32;
    __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
};
template <>
struct KBlock<bf16> {
    static constexpr int kK = 32;
    __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
};
template <>
struct KBlock<float> {
    static constexpr int kK = 16;
    __device__ __forceinline__ static f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
        const f32x4 x = __builtin_bit_cast(f32x4, a), y = __builtin_bit_cast(f32x4, b);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(x[0], y[0], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(x[1], y[1], c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x4f32(x[2], y[2], c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x4f32(x[3], y[3], c, 0, 0, 0);
    }
};

// The direct-to-LDS kernels for large 16-bit problems (td_gemm_dma.hip): dtype kF16 or kBF16, K % 64 == 0,
// 16-byte aligned a and w; variant 14 (256 x 128 tiles, one per workgroup) or 18 (persistent 256 x 256 tiles, one
// workgroup per CU, for shapes gemm_persistent_fits accepts: M, NO >= 256, NO % 16 == 0 and NO <= 8192, 16-byte
// aligned c and bias, a head-major D a multiple of 16, M * K, NO * K and M * NO below 2^31).
bool gemm_persistent_fits(int dtype, const GemmParams& p);
int launch_gemm_dma(int dtype, GemmParams p, hipStream_t stream, int variant);

// The streaming kernel for narrow K (td_gemm_stream.hip): 16-bit, NO = 256, K = 128 or 256, 16-byte aligned a, w, c
// and bias (or no bias); a head-major output needs hm_D a multiple of 8.
bool gemm_stream_fits(int dtype, const GemmParams& p);
// w_stored: p.w is [K, 256] as its owner stores it (C = A . W) instead of [256, K]
int launch_gemm_stream(int dtype, GemmParams p, hipStream_t stream, bool w_stored = false);

}  // namespace td
