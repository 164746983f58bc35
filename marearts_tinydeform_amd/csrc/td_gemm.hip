// Project mode, first half: value[M, NO] = memory[M, K] . weight[NO, K]^T + bias[NO]
// (M = B*N tokens, K = C channels, NO = H*D), float32 accumulation, one rounding to the element type.
//
// gemm_mfma_kernel (half / bfloat16, K % 8 == 0, 16-byte aligned operands): 128 x 64 output tile per
// 256-thread workgroup, K in steps of 32 through double-buffered LDS; wavefront w owns rows 32w..32w+31 of the
// tile (2 x 4 tiles of v_mfma_f32_16x16x32). Tiles are numbered so that the N tiles of one M tile go to the same
// XCD (workgroups are dealt to the 8 XCDs round-robin), which keeps the memory rows in that XCD's L2.
// gemm_generic_kernel: any type/alignment (float, double, unaligned 16-bit); 64 x 64 tile, VALU FMAs.
#include "td_internal.h"

namespace td {
namespace {

constexpr int kXcds = 8;

struct GemmParams {
    const void* a;
    const void* w;
    const void* bias;
    void* c;
    int M, K, NO;
    int mt, nt;  // tile counts
    int per_xcd;
};

// Linear tile index for this workgroup; -1 when the workgroup has no tile.
__device__ __forceinline__ int tile_of(const GemmParams& p) {
    const int id = blockIdx.x;
    const int tile = (id % kXcds) * p.per_xcd + id / kXcds;
    return tile < p.mt * p.nt ? tile : -1;
}

template <typename T>
struct Mma16;
template <>
struct Mma16<f16> {
    typedef f16x8 frag;
    __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <>
struct Mma16<bf16> {
    typedef bf16x8 frag;
    __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

template <typename T>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmParams p) {
    constexpr int BM = 128, BN = 64, BK = 32, LDK = BK + 8;  // LDS row pitch in elements (80 bytes)
    using MM = Mma16<T>;
    using frag = typename MM::frag;
    __shared__ __align__(16) T As[2][BM * LDK];
    __shared__ __align__(16) T Bs[2][BN * LDK];

    const int tile = tile_of(p);
    if (tile < 0) return;
    const int m0 = (tile / p.nt) * BM, n0 = (tile % p.nt) * BN;
    const T* __restrict__ A = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    T* __restrict__ Cm = static_cast<T*>(p.c);
    const int M = p.M, K = p.K, NO = p.NO;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // global -> register staging: A tile = 512 chunks of 8 elements (2 per thread), B tile = 256 chunks
    u32x4 ra[2], rb;
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int cidx = tid + i * 256, row = cidx >> 2, kc = (cidx & 3) * 8;
            const int gm = m0 + row, gk = k0 + kc;
            ra[i] = u32x4{0u, 0u, 0u, 0u};
            if (gm < M && gk < K) ra[i] = *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(gm) * K + gk);
        }
        const int row = tid >> 2, kc = (tid & 3) * 8;
        const int gn = n0 + row, gk = k0 + kc;
        rb = u32x4{0u, 0u, 0u, 0u};
        if (gn < NO && gk < K) rb = *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(gn) * K + gk);
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int cidx = tid + i * 256, row = cidx >> 2, kc = (cidx & 3) * 8;
            *reinterpret_cast<u32x4*>(&As[buf][row * LDK + kc]) = ra[i];
        }
        const int row = tid >> 2, kc = (tid & 3) * 8;
        *reinterpret_cast<u32x4*>(&Bs[buf][row * LDK + kc]) = rb;
    };

    f32x4 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nk = (K + BK - 1) / BK;
    gload(0);
    sstore(0);
    __syncthreads();
    const int r16 = lane & 15, kg = (lane >> 4) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload((kt + 1) * BK);
        frag a[2], b[4];
#pragma unroll
        for (int i = 0; i < 2; ++i)
            a[i] = *reinterpret_cast<const frag*>(&As[cur][(wave * 32 + i * 16 + r16) * LDK + kg]);
#pragma unroll
        for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const frag*>(&Bs[cur][(j * 16 + r16) * LDK + kg]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = MM::mma(a[i], b[j], acc[i][j]);
        if (kt + 1 < nk) sstore(cur ^ 1);
        __syncthreads();
    }

    // epilogue: lane holds rows 4*(lane/16)+e of each 16x16 tile, column lane%16
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + j * 16 + r16;
        if (n >= NO) continue;
        const float bv = bias != nullptr ? static_cast<float>(bias[n]) : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + wave * 32 + i * 16 + (lane >> 4) * 4 + e;
                if (m < M) Cm[static_cast<size_t>(m) * NO + n] = static_cast<T>(acc[i][j][e] + bv);
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmParams p) {
    using A = typename AccOf<T>::type;
    constexpr int BT = 64, BK = 16;
    __shared__ A As[BK][BT + 1];
    __shared__ A Bs[BK][BT + 1];
    const int tile = tile_of(p);
    if (tile < 0) return;
    const int m0 = (tile / p.nt) * BT, n0 = (tile % p.nt) * BT;
    const T* __restrict__ Am = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    T* __restrict__ Cm = static_cast<T*>(p.c);
    const int M = p.M, K = p.K, NO = p.NO;
    const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
    A acc[4][4];
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j) acc[i][j] = 0;
    for (int k0 = 0; k0 < K; k0 += BK) {
        for (int e = tid; e < BT * BK; e += 256) {
            const int row = e / BK, k = e % BK;
            const int gm = m0 + row, gn = n0 + row, gk = k0 + k;
            As[k][row] = (gm < M && gk < K) ? cvt<A>(Am[static_cast<size_t>(gm) * K + gk]) : static_cast<A>(0);
            Bs[k][row] = (gn < NO && gk < K) ? cvt<A>(W[static_cast<size_t>(gn) * K + gk]) : static_cast<A>(0);
        }
        __syncthreads();
#pragma unroll 4
        for (int k = 0; k < BK; ++k) {
            A a[4], b[4];
            for (int i = 0; i < 4; ++i) a[i] = As[k][ty + 16 * i];
            for (int j = 0; j < 4; ++j) b[j] = Bs[k][tx + 16 * j];
            for (int i = 0; i < 4; ++i)
                for (int j = 0; j < 4; ++j) acc[i][j] = fma(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
    for (int j = 0; j < 4; ++j) {
        const int n = n0 + tx + 16 * j;
        if (n >= NO) continue;
        const A bv = bias != nullptr ? cvt<A>(bias[n]) : static_cast<A>(0);
        for (int i = 0; i < 4; ++i) {
            const int m = m0 + ty + 16 * i;
            if (m < M) Cm[static_cast<size_t>(m) * NO + n] = static_cast<T>(acc[i][j] + bv);
        }
    }
}

template <typename T, bool MFMA>
int go(GemmParams p, int bm, int bn, hipStream_t stream) {
    p.mt = (p.M + bm - 1) / bm;
    p.nt = (p.NO + bn - 1) / bn;
    const int64_t tiles = static_cast<int64_t>(p.mt) * p.nt;
    p.per_xcd = static_cast<int>((tiles + kXcds - 1) / kXcds);
    const unsigned grid = static_cast<unsigned>(static_cast<int64_t>(p.per_xcd) * kXcds);
    if constexpr (MFMA) {
        hipLaunchKernelGGL((gemm_mfma_kernel<T>), dim3(grid), dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL((gemm_generic_kernel<T>), dim3(grid), dim3(256), 0, stream, p);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "value_proj launch failed: %s", hipGetErrorString(e));
}

template <typename T>
int launch_t(GemmParams p, hipStream_t stream, int force_generic) {
    if constexpr (sizeof(T) == 2) {
        const uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w);
        if (!force_generic && p.K % 8 == 0 && al % 16 == 0) return go<T, true>(p, 128, 64, stream);
    }
    return go<T, false>(p, 64, 64, stream);
}

}  // namespace

int launch_value_proj(int dtype, const void* a, const void* w, const void* bias, void* c, int64_t M, int64_t K,
                      int64_t NO, hipStream_t stream, int force_generic) {
    GemmParams p{a, w, bias, c, static_cast<int>(M), static_cast<int>(K), static_cast<int>(NO), 0, 0, 0};
    switch (dtype) {
        case kF32: return launch_t<float>(p, stream, force_generic);
        case kF16: return launch_t<f16>(p, stream, force_generic);
        case kBF16: return launch_t<bf16>(p, stream, force_generic);
        case kF64: return launch_t<double>(p, stream, force_generic);
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
}

}  // namespace td
