// The register-operand MFMA GEMM of the value projection as a device body: GemmMfmaTile<...>::run computes one
// output tile with the LDS its caller provides (kLds bytes, 16-byte aligned). gemm_mfma_kernel (td_gemm.hip) runs it
// for the tile tile_of gives its workgroup; the training backward (td_backward.hip) runs it beside the weight
// gradient in one launch.
#pragma once

#include "td_gemm.h"

namespace td {

// MFMA GEMM, both operands K-contiguous (C = A . W^T). WM x WN wavefronts per workgroup; wavefront (wm, wn) owns a
// TM x TN grid of 16x16 output tiles. K advances in chunks of NKB 16-byte blocks:
//   A  each wavefront loads its own rows straight from global memory into MFMA fragments (one chunk ahead);
//   W  the workgroup stages the BN x chunk slice in LDS (two buffers, filled from registers one chunk ahead).
// STAGES = 2 overlaps the next chunk's loads with this chunk's MFMAs; STAGES = 1 (one LDS buffer) suits K that fits
// one chunk, where the whole product costs a single round trip to memory.
// Epilogue: bias, one rounding to T, the tile transposed through LDS and written with 16-byte stores.
// DUAL: C = A . W^T + A2 . W^T + bias with A2 the same shape as A (two MFMAs per block; the sum A + A2 is never
// rounded to T). F32OUT: C is float32, the accumulators stored unrounded.
// WT (16-bit types): W is given as stored by its owner, [K, NO] with NO contiguous (C = A . W), so no transposed copy
// is needed: the K x BN slice is staged as K rows (pitch BN + 16 elements: measured at the RT-DETR training step's
// input gradient against BN + 4 and BN + 8, 57.1 and 56.3 against 56.1 us), and each B fragment (8 consecutive k
// of one column) is read by two LDS transpose reads (ds_read_b64_tr_b16: within each 16 lanes, lane i receives
// element i % 4 of the 8-byte pieces the lanes i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4 point at, so lanes
// pointing at rows k .. k + 3, columns c + 4 (lane % 4) give lane i the four k of column c + i).
template <typename T, int WM, int WN, int TM, int TN, int NKB, int STAGES, bool DUAL = false, bool F32OUT = false,
          bool WT = false>
struct GemmMfmaTile {
    using O = typename std::conditional<F32OUT, float, T>::type;  // output element
    static constexpr int NTH = WM * WN * kWave;
    static constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per 16 bytes
    static constexpr int EO = 16 / static_cast<int>(sizeof(O));  // output elements per 16 bytes
    static constexpr int KBK = KBlock<T>::kK;                   // K per 16-byte block (4 lane groups)
    static constexpr int KC = NKB * KBK;                         // K per chunk
    static constexpr int BM = WM * TM * 16, BN = WN * TN * 16;
    static constexpr int LDK = KC + E;                           // LDS pitch (elements) of a staged W row
    static constexpr int LDN = BN + 16;                          // WT: LDS pitch (elements) of a staged k row
    static constexpr int B_CHUNKS = BN * KC / E;                 // 16-byte pieces of one staged W slice
    static constexpr int B_PER_T = (B_CHUNKS + NTH - 1) / NTH;
    static constexpr int LDC = BN + EO;                          // LDS pitch of the output tile
    static_assert(!WT || sizeof(T) == 2, "the transposed-W form reads 16-bit fragments");
    static constexpr size_t kStage =
        WT ? static_cast<size_t>(KC) * LDN * sizeof(T) : static_cast<size_t>(BN) * LDK * sizeof(T);
    static constexpr size_t kOut = static_cast<size_t>(BM) * LDC * sizeof(O);
    static constexpr size_t kLds = STAGES * kStage > kOut ? STAGES * kStage : kOut;

    __device__ __forceinline__ static void run(const GemmParams& p, int tile, unsigned char* lds) {
        auto stage = [&](int i) { return reinterpret_cast<T*>(lds + (STAGES == 2 ? (i & 1) * kStage : 0)); };

        const int m0 = (tile / p.nt) * BM, n0 = (tile % p.nt) * BN;
        const T* __restrict__ A = static_cast<const T*>(p.a);
        const T* __restrict__ A2 = static_cast<const T*>(p.a2);
        const T* __restrict__ W = static_cast<const T*>(p.w);
        const T* __restrict__ bias = static_cast<const T*>(p.bias);
        O* __restrict__ Cm = static_cast<O*>(p.c);
        const int M = p.M, K = p.K, NO = p.NO;

        const int tid = threadIdx.x, wave = tid / kWave, lane = tid & (kWave - 1);
        const int wm = wave / WN, wn = wave % WN;
        const int r16 = lane & 15, kg = lane >> 4;
        const u32x4 zero = {0u, 0u, 0u, 0u};

        // A fragments of one chunk: row m0 + wm*TM*16 + i*16 + r16, k = k0 + j*KBK + kg*E (and the same of A2)
        constexpr int NA = DUAL ? 2 : 1;
        auto load_a = [&](u32x4 (&a)[NA][TM][NKB], int k0) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int m = m0 + (wm * TM + i) * 16 + r16;
#pragma unroll
                for (int j = 0; j < NKB; ++j) {
                    const int k = k0 + j * KBK + kg * E;
                    const bool in = m < M && k < K;
                    a[0][i][j] = in ? *reinterpret_cast<const u32x4*>(A + static_cast<size_t>(m) * K + k) : zero;
                    if constexpr (DUAL)
                        a[NA - 1][i][j] =
                            in ? *reinterpret_cast<const u32x4*>(A2 + static_cast<size_t>(m) * K + k) : zero;
                }
            }
        };
        u32x4 rb[B_PER_T];
        auto load_b = [&](int k0) {
#pragma unroll
            for (int u = 0; u < B_PER_T; ++u) {
                const int c = tid + u * NTH;
                if constexpr (WT) {  // piece c: k row c / (BN / E), columns (c % (BN / E)) * E .. + E - 1
                    const int kk = c / (BN / E), nn = (c % (BN / E)) * E;
                    const int n = n0 + nn, k = k0 + kk;
                    rb[u] = (c < B_CHUNKS && n < NO && k < K)
                                ? *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(k) * NO + n)
                                : zero;
                } else {
                    const int row = c / (KC / E), kc = (c % (KC / E)) * E;
                    const int n = n0 + row, k = k0 + kc;
                    rb[u] = (c < B_CHUNKS && n < NO && k < K)
                                ? *reinterpret_cast<const u32x4*>(W + static_cast<size_t>(n) * K + k)
                                : zero;
                }
            }
        };
        auto store_b = [&](T* buf) {
#pragma unroll
            for (int u = 0; u < B_PER_T; ++u) {
                const int c = tid + u * NTH;
                if (c < B_CHUNKS) {
                    if constexpr (WT) {
                        const int kk = c / (BN / E), nn = (c % (BN / E)) * E;
                        *reinterpret_cast<u32x4*>(buf + kk * LDN + nn) = rb[u];
                    } else {
                        const int row = c / (KC / E), kc = (c % (KC / E)) * E;
                        *reinterpret_cast<u32x4*>(buf + row * LDK + kc) = rb[u];
                    }
                }
            }
        };

        f32x4 acc[TM][TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

        const int nc = (K + KC - 1) / KC;
        auto mma_chunk = [&](const u32x4 (&a)[NA][TM][NKB], const T* bs) {
#pragma unroll
            for (int j = 0; j < NKB; ++j) {
                u32x4 b[TN];
#pragma unroll
                for (int t = 0; t < TN; ++t) {
                    if constexpr (WT) {  // k rows j * KBK + 8 kg + lane16 / 4 (+ 4), columns 4 (lane16 % 4) on
                        using v4s = short __attribute__((ext_vector_type(4)));
                        using lds_v4s = __attribute__((address_space(3))) v4s;
                        const T* q = bs + (j * KBK + kg * 8 + (r16 >> 2)) * LDN + (wn * TN + t) * 16 + 4 * (r16 & 3);
                        const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(q));
                        const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(q + 4 * LDN));
                        b[t] = __builtin_bit_cast(u32x4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    } else {
                        b[t] = *reinterpret_cast<const u32x4*>(bs + ((wn * TN + t) * 16 + r16) * LDK + j * KBK +
                                                               kg * E);
                    }
                }
#pragma unroll
                for (int o = 0; o < NA; ++o)
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int t = 0; t < TN; ++t) acc[i][t] = KBlock<T>::mma(a[o][i][j], b[t], acc[i][t]);
            }
        };
        if constexpr (STAGES == 1) {
            u32x4 a_cur[NA][TM][NKB];
            for (int c = 0; c < nc; ++c) {
                load_a(a_cur, c * KC);
                load_b(c * KC);
                if (c > 0) __syncthreads();  // every wavefront is done with the previous chunk's slice
                store_b(stage(0));
                __syncthreads();
                mma_chunk(a_cur, stage(0));
            }
            __syncthreads();
        } else {
            u32x4 a_cur[NA][TM][NKB], a_next[NA][TM][NKB];
            load_a(a_cur, 0);
            load_b(0);
            store_b(stage(0));
            __syncthreads();
            for (int c = 0; c < nc; ++c) {
                const bool more = c + 1 < nc;
                if (more) {
                    load_a(a_next, (c + 1) * KC);
                    load_b((c + 1) * KC);
                }
                mma_chunk(a_cur, stage(c));
                if (more) store_b(stage(c + 1));
                __syncthreads();
                if (more) {
#pragma unroll
                    for (int o = 0; o < NA; ++o)
#pragma unroll
                        for (int i = 0; i < TM; ++i)
#pragma unroll
                            for (int j = 0; j < NKB; ++j) a_cur[o][i][j] = a_next[o][i][j];
                }
            }
        }

        // epilogue through LDS (every wavefront has passed the last barrier, so the W buffers are free)
        O* Ct = reinterpret_cast<O*>(lds);
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const int nl = (wn * TN + t) * 16 + r16;
            const float bv = (bias != nullptr && n0 + nl < NO) ? static_cast<float>(bias[n0 + nl]) : 0.f;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    Ct[((wm * TM + i) * 16 + kg * 4 + e) * LDC + nl] = static_cast<O>(acc[i][t][e] + bv);
        }
        __syncthreads();
        const bool vec_ok = NO % EO == 0 && (reinterpret_cast<uintptr_t>(Cm) % 16) == 0;
        for (int c = tid; c < BM * (BN / EO); c += NTH) {
            const int row = c / (BN / EO), col = (c % (BN / EO)) * EO;
            const int m = m0 + row, n = n0 + col;
            if (m >= M || n >= NO) continue;
            const O* src = Ct + row * LDC + col;
            O* dst = Cm + out_index(p, m, n);
            if (vec_ok && n + EO <= NO) {
                *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
            } else {
                for (int e = 0; e < EO && n + e < NO; ++e) dst[e] = src[e];
            }
        }
    }
};

}  // namespace td
