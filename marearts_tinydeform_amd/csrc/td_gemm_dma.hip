// Value projection for large 16-bit problems: value[M, NO] = memory[M, K] . weight[NO, K]^T + bias[NO] on MFMA,
// operands streamed into LDS by direct global-to-LDS loads. Built with -mllvm -amdgpu-mfma-vgpr-form=1 (accumulators
// in architectural VGPRs): in the accumulator-register form the compiler routes each MFMA's accumulator through a
// temporary, extra moves and hazard NOPs in the inner loop.
#include "td_gemm.h"

namespace td {
namespace {

// Compiler scheduling fence: no instruction moves across.
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// 16 bytes per lane from global memory into LDS at (wavefront-uniform) dst + 16 * lane.
__device__ __forceinline__ void load_lds16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// Slot swizzle g of a staged row, from the row's index within its 16-row group.
__device__ __forceinline__ int swz(int r) { return ((r >> 1 ^ r >> 3) & 1) | (r & 4) >> 1; }

// Wait until at most VM vector-memory loads of this wavefront are in flight and its LDS reads are done, then meet
// the workgroup at a barrier, without the fence of __syncthreads (which would drain every outstanding load). The
// s_waitcnt builtin (unlike inline assembly) is seen by the compiler's own wait insertion, the empty asm with a
// memory clobber keeps memory accesses from moving across, and the scheduling barriers keep everything else in
// place. Encoding (gfx9): vmcnt in bits 3:0 and 15:14, expcnt 6:4 (7 = no wait), lgkmcnt 11:8.
template <int VM>
__device__ __forceinline__ void meet() {
    static_assert(VM >= 0 && VM <= 63, "vmcnt range");
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// 256 x BN tiles (BN = 64 * WN), 2 x WN wavefronts, each owning 128 x 64 of the tile (8 x 4 MFMA tiles of 16 x 16:
// 128 accumulators in VGPRs, two wavefronts per SIMD). Against 128 x 128 tiles this halves (BN = 128) or quarters
// (BN = 256) the L2 -> CU operand traffic per flop.
//
// K streams through a ring of STAGES LDS buffers, STAGES - 1 chunks of 32 ahead of the MFMAs, by direct
// global-to-LDS loads (global_load_lds_dwordx4: lane i's 16 bytes land at the wavefront's LDS base + 16 i), so the
// staging costs no registers and no LDS store instructions. The compiler does not track these loads against LDS
// reads, so the kernel orders them itself (meet()).
//
// LDS layout of a staged operand: [rows][4 slots of 16 bytes]; row r's K piece kc (8 elements) sits in slot
// kc ^ g(r) with g(r) = ((r >> 1 ^ r >> 3) & 1) | (r & 4) >> 1. A fragment read takes one kc from 16 consecutive rows;
// with this g the 16 rows land in 16 distinct 16-byte bank groups of a 256-byte window, and each half (8 rows) in 8
// distinct groups of a 128-byte window, so the read is conflict-free whether the LDS serves 16 or 8 lanes of a
// 16-byte read per cycle. The swizzle is applied on the source side: the lane whose LDS slot is s loads piece
// s ^ g(row). Rows past M or NO load the last valid row (their results are never stored), so no load is predicated.
template <typename T, int WN, int STAGES>
__global__ __launch_bounds__(128 * WN) __attribute__((amdgpu_waves_per_eu(2))) void gemm_dma_kernel(GemmParams p) {
    constexpr int TN = 4;
    constexpr int NTH = 128 * WN, WAVES = 2 * WN;
    constexpr int BM = 256, BN = 16 * TN * WN, KC = 32;  // elements; one 16x16x32 MFMA step per chunk
    constexpr int TM = 8, WTN = 16 * TN;                 // 16 x 16 tiles per wavefront; wavefront tile width
    constexpr int ROW_BYTES = KC * 2;               // 64
    constexpr int A_BYTES = BM * ROW_BYTES, B_BYTES = BN * ROW_BYTES;
    constexpr int STAGE_BYTES = A_BYTES + B_BYTES;
    constexpr int A_LOADS = BM / 16 / WAVES, B_LOADS = BN / 16 / WAVES;  // 1 KB wavefront loads per chunk
    constexpr int LOADS = A_LOADS + B_LOADS;
    static_assert(LOADS * (STAGES - 1) <= 63 && STAGES >= 2, "vmcnt range");
    extern __shared__ __align__(16) unsigned char lds[];

    const int tile = tile_of(p);
    if (tile < 0) return;
    const int m0 = (tile / p.nt) * BM, n0 = (tile % p.nt) * BN;
    const T* __restrict__ A = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const int M = p.M, K = p.K, NO = p.NO;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave / WN, wn = wave % WN;
    const int r16 = lane & 15, kg = lane >> 4;

    // load sources: wavefront w's load i of an operand fills rows (w * X_LOADS + i) * 16 .. + 16 of the stage;
    // lane = 4 * (row % 16) + slot, and g(row) depends on row % 16 = lane >> 2 only
    const int piece = ((lane & 3) ^ swz(lane >> 2)) * 8;
    const T* a_src[A_LOADS];
    const T* b_src[B_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        int m = m0 + (wave * A_LOADS + i) * 16 + (lane >> 2);
        m = m < M ? m : M - 1;
        a_src[i] = A + static_cast<size_t>(m) * K + piece;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        int n = n0 + (wave * B_LOADS + i) * 16 + (lane >> 2);
        n = n < NO ? n : NO - 1;
        b_src[i] = W + static_cast<size_t>(n) * K + piece;
    }
    // One group of loads per step, always: chunk c into stage c % STAGES, where c past the last chunk re-loads the
    // last chunk (an L2 hit) into a stage that is never read for the product again, so the number of loads in
    // flight, and with it every wait, is the same at each step.
    const int nc = K / KC;
    auto issue = [&](int c) {
        unsigned char* st = lds + (c % STAGES) * STAGE_BYTES;
        const int k = (c < nc ? c : nc - 1) * KC;
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            load_lds16(a_src[i] + k, st + (wave * A_LOADS + i) * 1024);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
            load_lds16(b_src[i] + k, st + A_BYTES + (wave * B_LOADS + i) * 1024);
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // fragment read offsets (bytes within a stage): row wm*128 + i*16 + r16 of A, wn*WTN + t*16 + r16 of B; the
    // slot swizzle depends on r16 only
    const int frag = r16 * ROW_BYTES + ((kg ^ swz(r16)) << 4);
    const int a_off = wm * 128 * ROW_BYTES + frag;
    const int b_off = A_BYTES + wn * WTN * ROW_BYTES + frag;
    auto read_frags = [&](int c, u32x4 (&xa)[TM], u32x4 (&xb)[TN]) {
        const unsigned char* st = lds + (c % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < TM; ++i) xa[i] = *reinterpret_cast<const u32x4*>(st + a_off + i * 16 * ROW_BYTES);
#pragma unroll
        for (int t = 0; t < TN; ++t) xb[t] = *reinterpret_cast<const u32x4*>(st + b_off + t * 16 * ROW_BYTES);
    };
    // Step c: wait for chunk c + 1 (the STAGES - 2 groups issued after it stay in flight) and for this wavefront's
    // fragment reads, meet the others (after which nobody reads chunk c's stage), refill that stage with chunk
    // c + STAGES, read chunk c + 1's fragments, then run chunk c's MFMAs on the fragments read one step earlier: the
    // MFMAs never wait on an LDS read. The last step's read of "chunk nc" reads a stage the tail re-load filled,
    // valid data that is never used, so every step is the same code.
    auto step = [&](int c, const u32x4 (&xa)[TM], const u32x4 (&xb)[TN], u32x4 (&ya)[TM], u32x4 (&yb)[TN]) {
        meet<LOADS * (STAGES - 2)>();
        issue(c + STAGES);
        read_frags(c + 1, ya, yb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int t = 0; t < TN; ++t) acc[i][t] = KBlock<T>::mma(xa[i], xb[t], acc[i][t]);
        // The next chunk's fragment reads and loads are not needed before the next step: spread them over the
        // MFMA stream (one read after each of the first MFMAs, one load after every second MFMA after that), so
        // their issue hides in the MFMA pipeline's shadow instead of delaying the first MFMA.
#pragma unroll
        for (int r = 0; r < TM + TN; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        }
#pragma unroll
        for (int r = 0; r < LOADS; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // vector memory read (the LDS load)
        }
        sched_fence();  // and the MFMAs ahead of the next step's barrier
    };
#pragma unroll
    for (int c = 0; c < STAGES; ++c) issue(c);
    meet<LOADS * (STAGES - 1)>();
    u32x4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    read_frags(0, fa0, fb0);
    for (int c = 0; c < nc; c += 2) {  // nc is even
        step(c, fa0, fb0, fa1, fb1);
        step(c + 1, fa1, fb1, fa0, fb0);
    }

    // epilogue: bias, one rounding, the tile transposed through LDS (once every wavefront's tail loads have landed
    // and its fragment reads are done), then 16-byte stores along rows
    meet<0>();
    constexpr int E = 8, LDC = BN + E;
    T* Ct = reinterpret_cast<T*>(lds);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        const int nl = wn * WTN + t * 16 + r16;
        const float bv = (bias != nullptr && n0 + nl < NO) ? static_cast<float>(bias[n0 + nl]) : 0.f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e)
                Ct[(wm * 128 + i * 16 + kg * 4 + e) * LDC + nl] = static_cast<T>(acc[i][t][e] + bv);
    }
    __syncthreads();
    T* __restrict__ Cm = static_cast<T*>(p.c);
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

template <typename T, int WN, int STAGES>
int go_dma(GemmParams p, hipStream_t stream) {
    constexpr int BN = 64 * WN;
    constexpr size_t stages = static_cast<size_t>(STAGES) * (256 + BN) * 64;
    constexpr size_t out = static_cast<size_t>(256) * (BN + 8) * sizeof(T);
    constexpr size_t lds = stages > out ? stages : out;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(gemm_dma_kernel<T, WN, STAGES>), hipFuncAttributeMaxDynamicSharedMemorySize,
        static_cast<int>(lds));
    if (attr != hipSuccess) return set_error(-3, "value_proj: LDS size attribute refused: %s", hipGetErrorString(attr));
    p.mt = (p.M + 255) / 256;
    p.nt = (p.NO + BN - 1) / BN;
    const int64_t tiles = static_cast<int64_t>(p.mt) * p.nt;
    p.per_xcd = static_cast<int>((tiles + kXcds - 1) / kXcds);
    const unsigned grid = static_cast<unsigned>(static_cast<int64_t>(p.per_xcd) * kXcds);
    hipLaunchKernelGGL((gemm_dma_kernel<T, WN, STAGES>), dim3(grid), dim3(128 * WN), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "value_proj launch failed: %s", hipGetErrorString(e));
}

// variants (td_gemm.hip lists them with the others): 14 = 256 x 128 tiles of 4 wavefronts, 16 = 256 x 256 tiles of
// 8 wavefronts; three LDS stages
template <typename T>
int launch_dma_t(GemmParams p, hipStream_t stream, int variant) {
    switch (variant) {
        case 14: return go_dma<T, 2, 3>(p, stream);
        case 16: return go_dma<T, 4, 3>(p, stream);
        default: return set_error(-1, "value_proj: unknown tile variant %d", variant);
    }
}

}  // namespace

int launch_gemm_dma(int dtype, GemmParams p, hipStream_t stream, int variant) {
    if (p.K % 64 != 0 || p.K == 0) return set_error(-1, "value_proj: tile variant %d needs K %% 64 == 0", variant);
    switch (dtype) {
        case kF16: return launch_dma_t<f16>(p, stream, variant);
        case kBF16: return launch_dma_t<bf16>(p, stream, variant);
        default: return set_error(-1, "value_proj: tile variant %d needs 16-bit operands", variant);
    }
}

}  // namespace td
