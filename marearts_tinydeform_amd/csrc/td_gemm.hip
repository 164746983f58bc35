// Project mode, first half: value[M, NO] = memory[M, K] . weight[NO, K]^T + bias[NO]
// (M = B*N tokens, K = C channels, NO = H*D), float32 accumulation, one rounding to the element type.
//
// gemm_mfma_kernel (half / bfloat16 / float, K a multiple of 16 bytes, 16-byte aligned operands): see below.
// Tiles are numbered so that the N tiles of one M tile go to the same XCD (workgroups are dealt to the 8 XCDs
// round-robin), which keeps the memory rows in that XCD's L2.
// gemm_generic_kernel: double, unaligned or odd-K operands; 64 x 64 tile, VALU FMAs.
#include "td_gemm_mfma.h"

namespace td {
namespace {

// MFMA GEMM, both operands K-contiguous (C = A . W^T): GemmMfmaTile (td_gemm_mfma.h) for this workgroup's tile.
template <typename T, int WM, int WN, int TM, int TN, int NKB, int STAGES, bool DUAL = false, bool F32OUT = false>
__global__ __launch_bounds__(WM* WN* kWave) void gemm_mfma_kernel(GemmParams p) {
    using G = GemmMfmaTile<T, WM, WN, TM, TN, NKB, STAGES, DUAL, F32OUT>;
    __shared__ __align__(16) unsigned char lds[G::kLds];
    const int tile = tile_of(p);
    if (tile < 0) return;
    G::run(p, tile, lds);
}
// MFMA GEMM for large problems: both operands staged through LDS (each element read from memory once per
// workgroup), two stages, WM x WN wavefronts each owning TM x TN 16x16 tiles (64 x 64 per wavefront), so a K block
// costs TM + TN fragment reads from LDS for TM * TN MFMAs.
template <typename T, int WM, int WN, int TM, int TN, int NKB>
__global__ __launch_bounds__(WM* WN* kWave) void gemm_lds_kernel(GemmParams p) {
    constexpr int NTH = WM * WN * kWave;
    constexpr int E = 16 / static_cast<int>(sizeof(T));
    constexpr int KBK = KBlock<T>::kK;
    constexpr int KC = NKB * KBK;
    constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    constexpr int LDK = KC + E;
    constexpr int A_CHUNKS = BM * KC / E, B_CHUNKS = BN * KC / E;
    constexpr int A_PER_T = (A_CHUNKS + NTH - 1) / NTH, B_PER_T = (B_CHUNKS + NTH - 1) / NTH;
    constexpr int LDC = BN + E;
    constexpr size_t kA = static_cast<size_t>(BM) * LDK * sizeof(T), kB = static_cast<size_t>(BN) * LDK * sizeof(T);
    constexpr size_t kStage = kA + kB;
    constexpr size_t kOut = static_cast<size_t>(BM) * LDC * sizeof(T);
    constexpr size_t kLds = 2 * kStage > kOut ? 2 * kStage : kOut;
    __shared__ __align__(16) unsigned char lds[kLds];
    auto as = [&](int i) { return reinterpret_cast<T*>(lds + (i & 1) * kStage); };
    auto bs = [&](int i) { return reinterpret_cast<T*>(lds + (i & 1) * kStage + kA); };

    const int tile = tile_of(p);
    if (tile < 0) return;
    const int m0 = (tile / p.nt) * BM, n0 = (tile % p.nt) * BN;
    const T* __restrict__ A = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    T* __restrict__ Cm = static_cast<T*>(p.c);
    const int M = p.M, K = p.K, NO = p.NO;
    const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15, kg = lane >> 4;
    const u32x4 zero = {0u, 0u, 0u, 0u};

    u32x4 ra[A_PER_T], rb[B_PER_T];
    auto load = [&](int k0) {
#pragma unroll
        for (int u = 0; u < A_PER_T; ++u) {
            const int c = tid + u * NTH, row = c / (KC / E), kc = (c % (KC / E)) * E;
            const int m = m0 + row, k = k0 + kc;
            ra[u] = (c < A_CHUNKS && m < M && k < K) ? *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(m) * K + k)
                                                     : zero;
        }
#pragma unroll
        for (int u = 0; u < B_PER_T; ++u) {
            const int c = tid + u * NTH, row = c / (KC / E), kc = (c % (KC / E)) * E;
            const int n = n0 + row, k = k0 + kc;
            rb[u] = (c < B_CHUNKS && n < NO && k < K) ? *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(n) * K + k)
                                                      : zero;
        }
    };
    auto store = [&](int stage) {
        T* a = as(stage);
        T* b = bs(stage);
#pragma unroll
        for (int u = 0; u < A_PER_T; ++u) {
            const int c = tid + u * NTH;
            if (c < A_CHUNKS) *reinterpret_cast<u32x4*>(a + (c / (KC / E)) * LDK + (c % (KC / E)) * E) = ra[u];
        }
#pragma unroll
        for (int u = 0; u < B_PER_T; ++u) {
            const int c = tid + u * NTH;
            if (c < B_CHUNKS) *reinterpret_cast<u32x4*>(b + (c / (KC / E)) * LDK + (c % (KC / E)) * E) = rb[u];
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int nc = (K + KC - 1) / KC;
    load(0);
    store(0);
    __syncthreads();
    for (int c = 0; c < nc; ++c) {
        const bool more = c + 1 < nc;
        if (more) load((c + 1) * KC);
        const T* a = as(c);
        const T* b = bs(c);
#pragma unroll
        for (int j = 0; j < NKB; ++j) {
            u32x4 fa[TM], fb[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i)
                fa[i] = *reinterpret_cast<const u32x4*>(a + ((wm * TM + i) * 16 + r16) * LDK + j * KBK + kg * E);
#pragma unroll
            for (int t = 0; t < TN; ++t)
                fb[t] = *reinterpret_cast<const u32x4*>(b + ((wn * TN + t) * 16 + r16) * LDK + j * KBK + kg * E);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int t = 0; t < TN; ++t) acc[i][t] = KBlock<T>::mma(fa[i], fb[t], acc[i][t]);
        }
        if (more) store(c + 1);
        __syncthreads();
    }

    T* Ct = reinterpret_cast<T*>(lds);
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        const int nl = (wn * TN + t) * 16 + r16;
        const float bv = (bias != nullptr && n0 + nl < NO) ? static_cast<float>(bias[n0 + nl]) : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Ct[((wm * TM + i) * 16 + kg * 4 + e) * LDC + nl] = static_cast<T>(acc[i][t][e] + bv);
    }
    __syncthreads();
    const bool vec_ok = NO % E == 0 && (reinterpret_cast<uintptr_t>(Cm) % 16) == 0;
    for (int c = tid; c < BM * (BN / E); c += NTH) {
        const int row = c / (BN / E), col = (c % (BN / E)) * E;
        const int m = m0 + row, n = n0 + col;
        if (m >= M || n >= NO) continue;
        const T* src = Ct + row * LDC + col;
        T* dst = Cm + out_index(p, m, n);
        if (vec_ok && n + E <= NO) {
            *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
        } else {
            for (int e = 0; e < E && n + e < NO; ++e) dst[e] = src[e];
        }
    }
}

// VALU GEMM for float64, odd K and unaligned operands: 64 x 64 tiles, K in blocks of 16 through LDS.
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
            if (m < M) Cm[out_index(p, m, n)] = static_cast<T>(acc[i][j] + bv);
        }
    }
}

template <typename Kernel>
int go(Kernel kernel, GemmParams p, int bm, int bn, int threads, hipStream_t stream) {
    p.mt = (p.M + bm - 1) / bm;
    p.nt = (p.NO + bn - 1) / bn;
    const int64_t tiles = static_cast<int64_t>(p.mt) * p.nt;
    p.per_xcd = static_cast<int>((tiles + kXcds - 1) / kXcds);
    const unsigned grid = static_cast<unsigned>(static_cast<int64_t>(p.per_xcd) * kXcds);
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), 0, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "value_proj launch failed: %s", hipGetErrorString(e));
}

template <typename T, int WM, int WN, int TM, int TN, int NKB>
int go_lds(GemmParams p, hipStream_t stream) {
    return go(gemm_lds_kernel<T, WM, WN, TM, TN, NKB>, p, WM * TM * 16, WN * TN * 16, WM * WN * kWave, stream);
}

template <typename T, int WM, int WN, int TM, int TN, int NKB, int STAGES>
int go_mfma(GemmParams p, hipStream_t stream) {
    return go(gemm_mfma_kernel<T, WM, WN, TM, TN, NKB, STAGES>, p, WM * TM * 16, WN * TN * 16, WM * WN * kWave,
              stream);
}

// Kernel by problem size: the tile variants the size rule picks (K per chunk = NKB 16-byte blocks, 32 elements each
// for 16-bit types, 16 for float32).
//   2  64 x 128  4 waves of 16 x 128, A fragments from memory, W through LDS, K chunks of 64/32, two stages
//   5  64 x 64   4 waves of 16 x 64, one chunk of 256/128 (K <= 256 for 16-bit: a single round trip), one stage
//   9  128 x 128 A and W through LDS (2 x 2 waves of 64 x 64), K chunks of 128/64
//   13 128 x 128 A and W through LDS, K chunks of 32/16
//   14 256 x 128 tiles fed by direct-to-LDS loads (td_gemm_dma.hip; 16-bit, K % 64 == 0)
//   18 persistent 256 x 256 tiles fed by direct-to-LDS loads, one workgroup per CU (td_gemm_dma.hip; 16-bit,
//      K % 64 == 0, gemm_persistent_fits)
//   22 the streaming kernel: a quarter of W in each wavefront's registers, token rows streamed through LDS
//      (td_gemm_stream.hip; 16-bit, NO = 256, K = 128 or 256)
//   23 64 x 32   4 waves of 16 x 32, one chunk of 256/128, one stage
//   24 32 x 32   2 waves of 16 x 32, one chunk of 256/128, one stage
//   25 64 x 64   4 waves of 16 x 64, K chunks of 128/64, two stages
//   0  gemm_generic_kernel (float64, odd K, A or W not 16-byte aligned)
//
// Measured on MI355X (16-bit):
//   256 outputs: the streaming kernel (22) from 14000 rows at K = 256 (M = 16384 8.3 µs against 9.1 for 25, M = 16800
//     9.1 against 11.2 for 13 and 12.2 for 25, M = 33600 12.2 against 15.4, M = 67200 17.6 against 23.5; it loses at
//     12000 rows, 7.8 against 7.4 for 25, and at 8400, 7.5 against 7.1), from 8000 rows at K = 128 (M = 8400 5.4
//     against 5.6 for 25, M = 16384 6.1 against 7.0);
//   deep K (K >= 512, K % 64 == 0) on a grid of at least 200 tiles of 256 x 128, or more than one round (256) of
//     128 x 128 tiles, or from 8000 rows: the direct-to-LDS kernels, persistent 256 x 256 tiles (18) from 120 of
//     them, else 256 x 128 (14) (C = 1024: M = 43520 87-89 µs for 18 against 97-100 for the same tiles one per
//     workgroup and 122 for 13; M = 8400 28.5 against 32.7 for 14; K = NO = 512: M = 50400 35.8 against 42.9, M = 16800 18.9 against
//     21.7; below 120 tiles 14 wins, M = 8400 14.2 against 16.6; M = 21760, K = NO = 1024 54-55 for both;
//     M = 7200 23.6 for 14 against 29.2 for 13; M = 6000 23.2 against 35.3 for 9; K = 512, NO = 256: M = 8400 14.4
//     against 22.1; K = NO = 768: M = 8400 19.3 against 28.8);
//   smaller grids by their count of 64 x 64 tiles:
//     K <= 256: up to 300 tiles 32 x 32 (24) (NO = 256: M = 300 3.3 against 4.5 for 64 x 64 one-chunk tiles, M = 2400
//       4.5 against 4.7), up to 1100 64 x 64 with two-stage K chunks of 128 (25) (M = 8400 7.2 against 7.8,
//       M = 16384 9.5 against 10.0), else 13 (M = 30000 12.9);
//     K >= 512: under 64 tiles 32 x 32 (24) (M = 100, K = NO = 1024: 6.5 against 10.2), under 128 64 x 32 (23)
//       (M = 300: 8.0 against 10.2), under 512 two-stage 64 x 64 (25) (M = 600: 10.0 against 10.4, M = 1800: 13.2
//       against 14.2), then both operands through LDS with K chunks of 128 (9) while under 512 tiles of 128 x 128
//       (M = 3600: 19.4 against 25.9; against the direct-to-LDS kernel, K = NO = 512: M = 2400 8.1 against 13.1,
//       M = 4800 11.5 against 13.6; K = NO = 1024: M = 1800 12.8 against 20.0, M = 3600 18.9 against 21.9), else 13.
// float32 (MFMA-bound: v_mfma_f32_16x16x4_f32), by the count of 64 x 64 tiles: K <= 256: up to 40 tiles 32 x 32 (24)
//   (K = NO = 256: M = 300 6.0 µs against 9.4 for 5), up to 100 64 x 32 (23) (M = 1200 6.8 against 9.5), up to 1100
//   two-stage 64 x 64 (25) (M = 2400 9.2 against 9.7, M = 8400 19.8 against 20.9), then 64 x 64 one-chunk tiles (5)
//   under 1024 tiles of 128 x 128 (M = 33600 54.4 against 56.2), else A direct in 64 x 128 tiles (2) (M = 67200: 93.5
//   against 96.4); K >= 512: two-stage 64 x 64 (25) under 512 tiles (M = 600, K = NO = 1024: 27.2 against 48.8 for
//   2), else 2.
int pick_variant(int dtype, const GemmParams& p) {
    if (dtype != kF32 && dtype != kF16 && dtype != kBF16) return 0;
    const int E = dtype == kF32 ? 4 : 8;
    const uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w);
    if (p.K % E != 0 || al % 16 != 0) return 0;
    const int64_t tiles_64 = ((p.M + 63) / 64) * static_cast<int64_t>((p.NO + 63) / 64);
    const int64_t tiles_128 = ((p.M + 127) / 128) * static_cast<int64_t>((p.NO + 127) / 128);
    if (dtype == kF32) {
        if (p.K <= 256) return tiles_64 <= 40 ? 24 : tiles_64 <= 100 ? 23 : tiles_64 <= 1100 ? 25 : tiles_128 < 1024 ? 5 : 2;
        return tiles_64 < 512 ? 25 : 2;
    }
    if (gemm_stream_fits(dtype, p) && p.M >= (p.K == 256 ? 14000 : 8000)) return 22;
    const int64_t tiles_256x128 = ((p.M + 255) / 256) * static_cast<int64_t>((p.NO + 127) / 128);
    const int64_t tiles_256 = ((p.M + 255) / 256) * static_cast<int64_t>((p.NO + 255) / 256);
    if (p.K >= 512 && p.K % 64 == 0 && (tiles_256x128 >= 200 || tiles_128 > 256 || p.M >= 8000))
        return tiles_256 >= 120 && gemm_persistent_fits(dtype, p) ? 18 : 14;
    if (p.K <= 256) return tiles_64 <= 300 ? 24 : tiles_64 <= 1100 ? 25 : 13;
    return tiles_64 < 64 ? 24 : tiles_64 < 128 ? 23 : tiles_64 < 512 ? 25 : tiles_128 < 512 ? 9 : 13;
}

template <typename T>
int launch_t(GemmParams p, hipStream_t stream, int variant) {
    constexpr int dt = std::is_same<T, float>::value ? kF32 : std::is_same<T, f16>::value ? kF16
                       : std::is_same<T, bf16>::value ? kBF16 : kF64;
    if constexpr (!std::is_same<T, double>::value) {
        switch (variant) {
            case 0: break;
            case 2: return go_mfma<T, 4, 1, 1, 8, 2, 2>(p, stream);
            case 5: return go_mfma<T, 4, 1, 1, 4, 8, 1>(p, stream);
            case 23: return go_mfma<T, 4, 1, 1, 2, 8, 1>(p, stream);
            case 24: return go_mfma<T, 2, 1, 1, 2, 8, 1>(p, stream);
            case 25: return go_mfma<T, 4, 1, 1, 4, 4, 2>(p, stream);
            case 9:
                if constexpr (sizeof(T) == 2) return go_lds<T, 2, 2, 4, 4, 4>(p, stream);
                break;
            case 13:
                if constexpr (sizeof(T) == 2) return go_lds<T, 2, 2, 4, 4, 1>(p, stream);
                break;
            case 14: case 18: return launch_gemm_dma(dt, p, stream, variant);
            case 22: return launch_gemm_stream(dt, p, stream);
            default: break;
        }
        if (variant != 0) return set_error(-1, "value_proj: no tile variant %d for this dtype", variant);
    }
    return go(gemm_generic_kernel<T>, p, 64, 64, 256, stream);
}

template <typename T>
int launch_proj_f32_t(GemmParams p, hipStream_t stream) {
    constexpr int E = 16 / static_cast<int>(sizeof(T));
    const uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w) |
                         reinterpret_cast<uintptr_t>(p.a2) | reinterpret_cast<uintptr_t>(p.c);
    if (p.K % E != 0 || al % 16 != 0) return 1;
    // 64 x 64 tiles, K in chunks of 256 (16-bit) / 128 (float32): the projections are short and wide
    if (p.a2 != nullptr)
        return go(gemm_mfma_kernel<T, 4, 1, 1, 4, 8, 1, true, true>, p, 64, 64, 4 * kWave, stream);
    return go(gemm_mfma_kernel<T, 4, 1, 1, 4, 8, 1, false, true>, p, 64, 64, 4 * kWave, stream);
}

}  // namespace

int launch_proj_f32(int dtype, const void* a, const void* a2, const void* w, const void* bias, float* c, int64_t M,
                    int64_t K, int64_t NO, hipStream_t stream) {
    GemmParams p{a, w, bias, c, static_cast<int>(M), static_cast<int>(K), static_cast<int>(NO), 0, 0, 0, a2};
    switch (dtype) {
        case kF32: return launch_proj_f32_t<float>(p, stream);
        case kF16: return launch_proj_f32_t<f16>(p, stream);
        case kBF16: return launch_proj_f32_t<bf16>(p, stream);
        default: return 1;
    }
}

int launch_value_proj(int dtype, const void* a, const void* w, const void* bias, void* c, int64_t M, int64_t K,
                      int64_t NO, hipStream_t stream, int hm_N, int hm_H) {
    GemmParams p{a, w, bias, c, static_cast<int>(M), static_cast<int>(K), static_cast<int>(NO), 0, 0, 0};
    if (hm_N > 0) {
        p.hm_N = hm_N;
        p.hm_D = static_cast<int>(NO) / hm_H;
        p.hm_ndiv = make_fastdiv(static_cast<uint32_t>(hm_N));
        p.hm_ddiv = make_fastdiv(static_cast<uint32_t>(p.hm_D));
    }
    const int variant = pick_variant(dtype, p);
    switch (dtype) {
        case kF32: return launch_t<float>(p, stream, variant);
        case kF16: return launch_t<f16>(p, stream, variant);
        case kBF16: return launch_t<bf16>(p, stream, variant);
        case kF64: return launch_t<double>(p, stream, variant);
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
}

int value_proj_plan(int dtype, const void* a, const void* w, const void* bias, const void* c, int64_t M, int64_t K,
                    int64_t NO, int hm_N, int hm_H) {
    GemmParams p{a, w, bias, const_cast<void*>(c), static_cast<int>(M), static_cast<int>(K), static_cast<int>(NO),
                 0, 0, 0};
    if (hm_N > 0) {
        p.hm_N = hm_N;
        p.hm_D = static_cast<int>(NO) / hm_H;
    }
    return pick_variant(dtype, p);
}

}  // namespace td
