// Streaming value projection for narrow K: value[M, 256] = memory[M, K] . W[256, K]^T + bias, K = 128 or 256,
// 16-bit operands (the C = 256 projections of RT-DETR, DINO and Deformable-DETR decoders).
//
// At K <= 256 the product is bound by HBM: each token row is read once (K * 2 bytes) and its value row written once
// (512 bytes), 128 flops per byte, below MI355X's ridge. A tiled GEMM spends a tile's short life (K / 32 chunks)
// on staging W and crossing barriers; this kernel instead keeps W resident and lets every wavefront stream:
//   * one workgroup per CU (persistent grid), W (64 or 128 KB) and the bias staged into LDS once;
//   * each workgroup owns an equal share of M and walks it in rounds of 4 x 32 tokens, one 32-token step per
//     wavefront, loading the token rows straight from HBM into MFMA fragments two steps ahead of the MFMAs (double
//     buffer, no barrier inside the loop, no LDS traffic for the tokens). A short remainder (at most 64 tokens at
//     K = 256, 32 at K = 128) goes through in steps that all four wavefronts take together, each computing a
//     quarter of the 256 channels, so it costs a quarter step per 32 tokens instead of a whole step; a longer one
//     is spread evenly, every wavefront walking a quarter of the share;
//   * the product is formed transposed, D = W . tokens^T on v_mfma_f32_16x16x32, so a lane's 4 accumulators are 4
//     output channels of one token. The W rows of the 16 x 16 output tiles are permuted so that tiles 2p and 2p + 1
//     give lane (r, kg) channels 32 p + 8 kg .. + 3 and + 4 .. + 7 of token r: 8 consecutive channels, one 16-byte
//     store (row 4 a + b of tile 2p + h is channel 32 p + 8 a + 4 h + b).
// LDS layout of W: [256 rows][K / 8 chunks of 16 bytes], chunk c of row n at slot c ^ key(n) with
// key(n) = ((n >> 1) & 12) | (n & 3), which differs across the 16 rows of one fragment read (one chunk each), so they
// fall in 16 distinct 16-byte bank groups.
#include <type_traits>

#include "td_gemm.h"

namespace td {
namespace {

constexpr int kStreamNO = 256;   // output columns
constexpr int kStreamWaves = 4;  // wavefronts per workgroup (one per SIMD)
constexpr int kStreamTM = 2;     // 16-token halves per step

template <typename T>
struct Out8 {
    T v[8];
};

// LDS slot key of W row n (see the layout above)
__device__ __forceinline__ int wkey(int n) { return ((n >> 1) & 12) | (n & 3); }

// 16 bytes per lane from global memory straight into LDS: lane i's bytes land at dst + 16 i (dst is the
// wavefront's base, the same for every lane)
__device__ __forceinline__ void load_lds16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

template <typename T, int KB, bool SPLIT>
__global__ __launch_bounds__(kStreamWaves* kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_stream_kernel(
    GemmParams p) {
    constexpr int NT = kStreamNO / 16;  // output tiles of 16 channels
    constexpr int CH = KB * 4;          // 16-byte chunks per row (K / 8)
    constexpr int TM = kStreamTM;
    static_assert(CH % 16 == 0, "the swizzle needs K a multiple of 128");
    extern __shared__ __align__(16) unsigned char smem[];
    u32x4* ws = reinterpret_cast<u32x4*>(smem);        // [256][CH]
    const T* bs = reinterpret_cast<const T*>(ws + kStreamNO * CH);  // [256] the bias in dtype

    const T* __restrict__ A = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    T* __restrict__ C = static_cast<T*>(p.c);
    const int M = p.M, K = p.K;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int r = lane & 15, kg = lane >> 4;

    // this workgroup's tokens [lo, hi): an equal share of M, taken one of two ways.
    //  * Rounds (SPLIT, and the share is whole rounds of 4 x 32 tokens plus a short remainder): step i < R is tokens
    //    lo + 128 i + 32 wave .. + 31, all 256 channels; each remainder step i >= R is tokens lo + 128 R + 32 (i - R)
    //    .. + 31 for every wavefront, channels 64 wave .. + 63 (tiles 4 wave .. + 3). Remainder steps pay a step's
    //    latency each for a quarter of its MFMAs: at K = 256 two of them beat a round, at K = 128 (half the MFMAs
    //    per step) only one does (80000 x 128: 16.1 against 14.7 µs with two).
    //  * Otherwise every wavefront walks an equal quarter [wlo, whi) of the share in steps of 32, all channels. A
    //    last round that only some wavefronts fill would leave the others idle and the first ones with more stores
    //    (80000 x 128: 16.3 against 14.7 µs).
    //  Without SPLIT the quarters are taken over the whole of M (the same split up to rounding).
    const int lo = static_cast<int>(static_cast<int64_t>(blockIdx.x) * M / gridDim.x);
    const int hi = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * M / gridDim.x);
    constexpr int kRound = 32 * kStreamWaves, kRemMax = KB == 8 ? 2 * 32 : 32;
    const int rem = (hi - lo) % kRound;
    const bool rounds = SPLIT && rem <= kRemMax;  // the same for the whole workgroup
    const int64_t nw = static_cast<int64_t>(gridDim.x) * kStreamWaves;
    const int64_t gw = static_cast<int64_t>(blockIdx.x) * kStreamWaves + wave;
    const int wlo = !SPLIT ? static_cast<int>(gw * M / nw) : rounds ? lo : lo + (hi - lo) * wave / kStreamWaves;
    const int whi = !SPLIT ? static_cast<int>((gw + 1) * M / nw)
                           : rounds ? hi : lo + (hi - lo) * (wave + 1) / kStreamWaves;
    const int R = rounds ? (hi - lo) / kRound : (whi - wlo + 31) / 32;  // steps over all 256 channels
    const int ns = rounds ? R + (rem + 31) / 32 : R;                  // steps of this wavefront
    const int mmax = whi > wlo ? whi - 1 : 0;                         // last row a load may touch
    auto tok = [&](int i) {
        i = i < ns ? i : ns - 1;
        if (!rounds) return wlo + 32 * i;
        return i < R ? lo + 32 * (kStreamWaves * i + wave) : lo + 32 * (kStreamWaves * R + i - R);
    };

    // token fragments of step i: lane (r, kg) holds token tok(i) + 16 s + r, k = 32 kb + 8 kg .. + 7. Rows past whi
    // read row whi - 1 (never stored) and a step past the last re-reads the last step (L2 hits), so every load is
    // unconditional and the compiler's wait counts stay exact.
    auto load = [&](u32x4 (&tf)[TM][KB], int i) {
        const int m0 = tok(i);
#pragma unroll
        for (int s = 0; s < TM; ++s) {
            int m = m0 + s * 16 + r;
            m = m < mmax ? m : mmax;
            const T* row = A + static_cast<size_t>(m) * K + kg * 8;
#pragma unroll
            for (int kb = 0; kb < KB; ++kb) tf[s][kb] = *reinterpret_cast<const u32x4*>(row + kb * 32);
        }
    };

    // The bias (wavefront 0) and W go into LDS by direct loads; the workgroup waits for them and meets before any
    // token is requested. Requesting the first steps' tokens ahead of the wait was slower (M = 88892: 24.7 against
    // 22.4 µs): every wavefront's 32 KB of token rows competed with W for the fabric, and W arrived last. Nothing else
    // writes LDS here: after a direct load the compiler orders any LDS store behind every outstanding load.
    // W: a wavefront's direct load fills 64 consecutive slots, so the swizzle is applied on the source side: the
    // lane that fills slot j of row n loads chunk j ^ key(n).
    static_assert(kStreamNO * sizeof(T) == 32 * 16, "the bias is 32 lanes x 16 bytes");
    if (bias != nullptr && wave == 0 && lane < 32) load_lds16(bias + lane * 8, const_cast<T*>(bs));
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order
    constexpr int WCH = kStreamNO * CH;
    constexpr int NU = WCH / (kStreamWaves * kWave);  // W pieces per wavefront
    static_assert(WCH % (kStreamWaves * kWave) == 0 && (NU & (NU - 1)) == 0, "W staging tiles the workgroup");
    // every workgroup stages the same 64 or 128 KB at the same moment: the CUs of one XCD start at different pieces
    // (workgroups are dealt to the XCDs round-robin), so their requests spread over the L2 channels
    const int rot = static_cast<int>(blockIdx.x / kXcds);
#pragma unroll
    for (int u = 0; u < NU; ++u) {  // a constant trip count, fully unrolled
        const int i0 = ((u + rot) & (NU - 1)) * kStreamWaves * kWave + wave * kWave;
        const int i = i0 + lane, n = i / CH, j = i - n * CH;
        load_lds16(W + static_cast<size_t>(n) * K + (j ^ wkey(n)) * 8, ws + i0);
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(7 << 4);  // vmcnt(0), lgkmcnt(0): W and the bias landed
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (whi <= wlo) return;
    u32x4 ta[TM][KB], tb[TM][KB];

    // the MFMAs of one step over NTW output tiles from tile t0 (all 16, or a wavefront's quarter)
    auto mma = [&](auto ntw, const u32x4 (&tf)[TM][KB], f32x4 (&acc)[TM][decltype(ntw)::value], int t0) {
        constexpr int NTW = decltype(ntw)::value;
#pragma unroll
        for (int s = 0; s < TM; ++s)
#pragma unroll
            for (int t = 0; t < NTW; ++t) acc[s][t] = f32x4{0.f, 0.f, 0.f, 0.f};
        // W fragment j = (kb, t): lane r reads row n = 32 (t / 2) + 8 (r / 4) + 4 (t % 2) + r % 4, chunk 4 kb + kg.
        // The fragments pass through a ring of DEPTH registers, each read DEPTH fragments ahead of its MFMAs; the
        // scheduling groups keep one LDS read between every two MFMAs.
        constexpr int J = KB * NTW, DEPTH = 8;
        const int rrow = 8 * (r >> 2) + (r & 3), rkey = wkey(rrow);  // wkey(n) is the same for every t
        auto rd = [&](int j) {
            const int kb = j / NTW, t = t0 + j - kb * NTW;
            const int n = 32 * (t >> 1) + 4 * (t & 1) + rrow;
            return ws[n * CH + ((kb * 4 + kg) ^ rkey)];
        };
        u32x4 ring[DEPTH];
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) ring[j] = rd(j);
        __builtin_amdgcn_sched_group_barrier(0x100, DEPTH, 0);  // the first DEPTH LDS reads
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int kb = j / NTW, t = j - kb * NTW;
            const u32x4 wf = ring[j % DEPTH];
            if (j + DEPTH < J) ring[j % DEPTH] = rd(j + DEPTH);
#pragma unroll
            for (int s = 0; s < TM; ++s) acc[s][t] = KBlock<T>::mma(wf, tf[s][kb], acc[s][t]);
            __builtin_amdgcn_sched_group_barrier(0x008, TM, 0);                  // TM MFMAs
            if (j + DEPTH < J) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // then one LDS read
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto store = [&](auto ntw, const f32x4 (&acc)[TM][decltype(ntw)::value], int m0, int t0) {
        // lane (r, kg) holds channels 32 p + 8 kg .. + 7 of token m0 + 16 s + r in tiles 2p (first 4) and 2p + 1
        constexpr int NTW = decltype(ntw)::value;
#pragma unroll
        for (int s = 0; s < TM; ++s) {
            const int m = m0 + s * 16 + r;
            if (m >= whi) continue;
            T* const row = C + out_row(p, m);
#pragma unroll
            for (int pp = 0; pp < NTW / 2; ++pp) {
                const int ch = 16 * t0 + 32 * pp + 8 * kg;
                Out8<T> bv = {};
                if (bias != nullptr) bv = __builtin_bit_cast(Out8<T>, *reinterpret_cast<const u32x4*>(bs + ch));
                Out8<T> o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    o.v[e] = static_cast<T>(acc[s][2 * pp][e] + cvt<float>(bv.v[e]));
                    o.v[4 + e] = static_cast<T>(acc[s][2 * pp + 1][e] + cvt<float>(bv.v[4 + e]));
                }
                *reinterpret_cast<u32x4*>(row + out_col(p, ch)) = __builtin_bit_cast(u32x4, o);
            }
        }
    };

    // Each step stores its outputs, then requests the next-but-one step's tokens into the registers its MFMAs have
    // just read. In the other order (tokens, then stores) the compiler's waits before the next MFMAs covered the
    // token requests just issued as well, and the two-step prefetch stopped overlapping (M = 88892: 25.0 against
    // 24.2 µs; 177784: 42.3 against 39.2). A step is a round step or a remainder step by a uniform branch inside
    // the one loop: a remainder loop of its own after this one made the compiler's waits at this loop's head cover
    // the loads just issued.
    using Full = std::integral_constant<int, NT>;
    using Quarter = std::integral_constant<int, NT / kStreamWaves>;
    auto step = [&](u32x4 (&x)[TM][KB], int i) {
        if (!SPLIT || i < R) {
            f32x4 acc[TM][NT];
            mma(Full{}, x, acc, 0);
            store(Full{}, acc, tok(i), 0);
        } else {
            f32x4 acc[TM][Quarter::value];
            mma(Quarter{}, x, acc, wave * Quarter::value);
            store(Quarter{}, acc, tok(i), wave * Quarter::value);
        }
        load(x, i + 2);
    };
    if constexpr (SPLIT) {
        load(ta, 0);
        load(tb, 1);
        for (int i = 0;;) {
            step(ta, i);
            if (++i >= ns) break;
            step(tb, i);
            if (++i >= ns) break;
        }
    } else {
        // the same walk by token offsets, the form the compiler schedules best when every step is whole (its one
        // full wait per two steps lands before the next tokens are requested, not after the stores: M = 88892
        // 23.3 against 24.3 µs)
        const int last = wlo + (whi - wlo - 1) / 32 * 32;  // first token of the last step
        auto load_at = [&](u32x4 (&tf)[TM][KB], int m0) {
            m0 = m0 < last ? m0 : last;
#pragma unroll
            for (int s = 0; s < TM; ++s) {
                int m = m0 + s * 16 + r;
                m = m < mmax ? m : mmax;
                const T* row = A + static_cast<size_t>(m) * K + kg * 8;
#pragma unroll
                for (int kb = 0; kb < KB; ++kb) tf[s][kb] = *reinterpret_cast<const u32x4*>(row + kb * 32);
            }
        };
        load_at(ta, wlo);
        load_at(tb, wlo + 32);
        f32x4 acc[TM][NT];
        for (int m0 = wlo;;) {
            mma(Full{}, ta, acc, 0);
            store(Full{}, acc, m0, 0);
            load_at(ta, m0 + 64);
            m0 += 32;
            if (m0 >= whi) break;
            mma(Full{}, tb, acc, 0);
            store(Full{}, acc, m0, 0);
            load_at(tb, m0 + 64);
            m0 += 32;
            if (m0 >= whi) break;
        }
    }
}

// compute units of the current device, asked once per device
template <typename T, int KB, bool SPLIT>
int go_stream(GemmParams p, int64_t grid, hipStream_t stream) {
    constexpr size_t lds = static_cast<size_t>(kStreamNO) * KB * 4 * 16 + kStreamNO * sizeof(T);
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(gemm_stream_kernel<T, KB, SPLIT>),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       static_cast<int>(lds));
    if (attr != hipSuccess) return set_error(-3, "value_proj: LDS size attribute refused: %s", hipGetErrorString(attr));
    hipLaunchKernelGGL((gemm_stream_kernel<T, KB, SPLIT>), dim3(static_cast<unsigned>(grid)), dim3(kStreamWaves * kWave),
                       lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "value_proj launch failed: %s", hipGetErrorString(e));
}

// One workgroup per CU, but at least one round of 4 x 32 tokens per workgroup (W is staged once per workgroup). The
// workgroups' shares differ by at most one token; the kernel with the remainder path (SPLIT) runs only when a share
// ends in a short remainder, since that path's code slows the other steps down (M = 88892: 24.0 against 23.3 µs).
template <typename T>
int stream_t(GemmParams p, hipStream_t stream) {
    int64_t grid = (static_cast<int64_t>(p.M) + 32 * kStreamWaves - 1) / (32 * kStreamWaves);
    const int cus = cu_count();
    if (grid > cus) grid = cus;
    if (grid < 1) grid = 1;
    const int64_t rem = (p.M / grid) % (32 * kStreamWaves);
    if (p.K == 256) return rem < 2 * 32 ? go_stream<T, 8, true>(p, grid, stream) : go_stream<T, 8, false>(p, grid, stream);
    return rem < 32 ? go_stream<T, 4, true>(p, grid, stream) : go_stream<T, 4, false>(p, grid, stream);
}

}  // namespace

// The bias is staged in LDS by a 16-byte direct load, so it must be 16-byte aligned like the other operands.
bool gemm_stream_fits(int dtype, const GemmParams& p) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w) |
                         reinterpret_cast<uintptr_t>(p.c) | reinterpret_cast<uintptr_t>(p.bias);
    return (dtype == kF16 || dtype == kBF16) && p.NO == kStreamNO && (p.K == 128 || p.K == 256) && p.M > 0 &&
           al % 16 == 0 && p.hm_D % 8 == 0;
}

int launch_gemm_stream(int dtype, GemmParams p, hipStream_t stream) {
    if (!gemm_stream_fits(dtype, p)) return set_error(-1, "value_proj: the streaming kernel does not take this shape");
    return dtype == kF16 ? stream_t<f16>(p, stream) : stream_t<bf16>(p, stream);
}

}  // namespace td
