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
};

// Linear tile index for this workgroup; -1 when the workgroup has no tile. Workgroups are dealt to the 8 XCDs
// round-robin, so consecutive tiles (the N tiles of one M tile) land on one XCD and share its L2.
__device__ __forceinline__ int tile_of(const GemmParams& p) {
    const int id = blockIdx.x;
    const int tile = (id % kXcds) * p.per_xcd + id / kXcds;
    return tile < p.mt * p.nt ? tile : -1;
}

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

// The direct-to-LDS kernel for large 16-bit problems (td_gemm_dma.hip): dtype kF16 or kBF16, K % 64 == 0,
// 16-byte aligned operands, variant 14..18.
int launch_gemm_dma(int dtype, GemmParams p, hipStream_t stream, int variant);

// The streaming kernel for narrow K (td_gemm_stream.hip): 16-bit, NO = 256, K = 128 or 256, 16-byte aligned a, w, c.
bool gemm_stream_fits(int dtype, const GemmParams& p);
int launch_gemm_stream(int dtype, GemmParams p, hipStream_t stream);

}  // namespace td
