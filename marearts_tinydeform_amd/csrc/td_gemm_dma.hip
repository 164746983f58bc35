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

// The 8-element vector of a 16-bit type.
template <typename T>
struct Vec8;
template <>
struct Vec8<f16> {
    using type = f16x8;
};
template <>
struct Vec8<bf16> {
    using type = bf16x8;
};

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
    static std::atomic<uint64_t> done{0};
    const hipError_t attr =
        allow_dynamic_lds(reinterpret_cast<const void*>(gemm_dma_kernel<T, WN, STAGES>), static_cast<int>(lds), done);
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

// Persistent form for many 256 x 256 tiles: the grid holds one workgroup per CU, and each workgroup walks its own
// tiles with one K-chunk pipeline across them, so the next tile's first chunks load while the current tile's last
// MFMAs run and its results are stored. 8 wavefronts as 2 (tokens) x 4 (channels), each owning 128 x 64 of the tile.
//
// The product is computed transposed (channels as the MFMA's rows, tokens as its columns): W stage position
// 64 wn + 16 t + r holds channel 64 wn + 16 (r >> 2) + 4 t + (r & 3) of the tile, so MFMA block t's output row
// 4 kg + e is channel 64 wn + 16 kg + 4 t + e and lane group kg ends with 16 consecutive channels of each of its
// tokens, which it stores from its accumulators as two 16-byte vectors: the epilogue needs no LDS, and the ring keeps
// streaming. Tiles are dealt per XCD (consecutive tiles share its L2); the G workgroups of an XCD take them
// round-robin with G a multiple of the channel-tile count, so each workgroup keeps one channel tile (and its bias) to
// the end. A last tile that would pass M (or NO) is moved back to end there: the rows it shares with its neighbour
// are computed twice, identically, and every load address is a per-lane constant plus a tile base in scalar
// registers. A tile's stores count in vmcnt too; the step after them still waits for exactly enough: loads complete in
// the order they were sent, so while any load of the awaited chunk is pending, every load sent after it is as well
// and the count stays above the wait's threshold, whether or not the stores have completed.
template <typename T, int STAGES>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2))) void gemm_dma_persistent_kernel(GemmParams p) {
    constexpr int KC = 32, ROW_BYTES = 64, BM = 256, BN = 256, WAVES = 8;
    constexpr int TM = 8, TN = 4;  // 16-token blocks, 16-channel blocks per wavefront
    constexpr int A_BYTES = BM * ROW_BYTES, STAGE_BYTES = (BM + BN) * ROW_BYTES;
    constexpr int A_LOADS = BM / 16 / WAVES, B_LOADS = BN / 16 / WAVES, LOADS = A_LOADS + B_LOADS;
    static_assert(LOADS * (STAGES - 1) <= 63 && STAGES >= 3 && A_LOADS == 2 && B_LOADS == 2, "tiling");
    extern __shared__ __align__(16) unsigned char lds[];

    const int M = p.M, K = p.K, NO = p.NO, nt = p.nt, ntiles = p.mt * p.nt;
    const int xcd = blockIdx.x % kXcds, G = gridDim.x / kXcds;
    const int first = xcd * p.per_xcd + static_cast<int>(blockIdx.x / kXcds);
    const int end = min((xcd + 1) * p.per_xcd, ntiles);
    if (first >= end) return;
    const int my_tiles = (end - first + G - 1) / G;
    const int n0 = min((first % nt) * BN, NO - BN), nc = K / KC;
    auto m0_of = [&](int k) { return min(((first + k * G) / nt) * BM, M - BM); };
    const T* __restrict__ A = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / 4, wn = wave % 4, r16 = lane & 15, kg = lane >> 4;

    // bias of this lane's 16 channels, loaded first (the first wait below covers it)
    const int nb = n0 + wn * 64 + kg * 16;
    u32x4 bias_raw[2] = {u32x4{0, 0, 0, 0}, u32x4{0, 0, 0, 0}};
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    if (bias != nullptr) {
        bias_raw[0] = *reinterpret_cast<const u32x4*>(bias + nb);
        bias_raw[1] = *reinterpret_cast<const u32x4*>(bias + nb + 8);
    }

    // Load sources (element offsets; the host keeps M * K and NO * K below 2^31): wavefront w's load i of an operand
    // fills stage rows (2 w + i) * 16 .. + 16, lane = 4 * (row % 16) + slot, slot s holding K piece s ^ g(row % 16).
    // Load i = 1 is load 0 sixteen token rows on, or four channels on (the next 16-position block of the stage).
    const int piece = ((lane & 3) ^ swz(lane >> 2)) * 8;
    const uint32_t a_lane = static_cast<uint32_t>((wave * 32 + (lane >> 2)) * K + piece);
    const int pos = wave * 32 + (lane >> 2), r = pos & 15;
    const uint32_t b_lane =
        static_cast<uint32_t>((n0 + (pos & ~63) + (r >> 2) * 16 + ((pos >> 4) & 3) * 4 + (r & 3)) * K + piece);
    const int a_step = 16 * K, b_step = 4 * K;
    // The load stream runs STAGES chunks ahead of the MFMAs through the workgroup's tiles; past the last chunk it
    // re-loads that chunk (an L2 hit) into a stage that is never read for the product, so every step sends one group.
    int is_k = 0, is_c = 0, stage_in = 0;
    const T* a_tile = A + static_cast<size_t>(m0_of(0)) * K;
    auto issue = [&]() {
        unsigned char* st = lds + stage_in * STAGE_BYTES;
        const T* ab = a_tile + is_c * KC;
        const T* wb = W + is_c * KC;
        load_lds16(ab + a_lane, st + wave * 2048);
        load_lds16(ab + a_step + a_lane, st + wave * 2048 + 1024);
        load_lds16(wb + b_lane, st + A_BYTES + wave * 2048);
        load_lds16(wb + b_step + b_lane, st + A_BYTES + wave * 2048 + 1024);
        stage_in = stage_in + 1 == STAGES ? 0 : stage_in + 1;
        if (++is_c == nc) {
            if (is_k + 1 < my_tiles) {
                is_c = 0;
                a_tile = A + static_cast<size_t>(m0_of(++is_k)) * K;
            } else {
                is_c = nc - 1;
            }
        }
    };

    f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int frag = r16 * ROW_BYTES + ((kg ^ swz(r16)) << 4);
    const int a_off = wm * 128 * ROW_BYTES + frag;
    const int b_off = A_BYTES + wn * 64 * ROW_BYTES + frag;
    int stage_out = 0;  // stage of the chunk whose fragments are read next
    auto read_frags = [&](u32x4 (&xa)[TM], u32x4 (&xb)[TN]) {
        const unsigned char* st = lds + stage_out * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < TM; ++i) xa[i] = *reinterpret_cast<const u32x4*>(st + a_off + i * 16 * ROW_BYTES);
#pragma unroll
        for (int t = 0; t < TN; ++t) xb[t] = *reinterpret_cast<const u32x4*>(st + b_off + t * 16 * ROW_BYTES);
        stage_out = stage_out + 1 == STAGES ? 0 : stage_out + 1;
    };

    // epilogue of tile k: bias, one rounding, two 16-byte stores per token (output offsets in 32 bits: the host keeps
    // M * NO below 2^31; channels nb + 8 follow nb in the output, NO and a head-major D being multiples of 16)
    T* __restrict__ Cm = static_cast<T*>(p.c);
    const uint32_t col = static_cast<uint32_t>(out_col(p, nb));
    auto epilogue = [&](int k) {
        using V8 = typename Vec8<T>::type;
        const V8 b0 = __builtin_bit_cast(V8, bias_raw[0]), b1 = __builtin_bit_cast(V8, bias_raw[1]);
        const int m0 = m0_of(k) + wm * 128 + r16;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const uint32_t o = static_cast<uint32_t>(out_row(p, m0 + i * 16)) + col;
            V8 v0, v1;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v0[e] = static_cast<T>(acc[i][0][e] + static_cast<float>(b0[e]));
                v0[4 + e] = static_cast<T>(acc[i][1][e] + static_cast<float>(b0[4 + e]));
                v1[e] = static_cast<T>(acc[i][2][e] + static_cast<float>(b1[e]));
                v1[4 + e] = static_cast<T>(acc[i][3][e] + static_cast<float>(b1[4 + e]));
            }
            *reinterpret_cast<u32x4*>(Cm + o) = __builtin_bit_cast(u32x4, v0);
            *reinterpret_cast<u32x4*>(Cm + o + 8) = __builtin_bit_cast(u32x4, v1);
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int t = 0; t < TN; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    // Step: wait for the next chunk (the STAGES - 2 groups sent after it stay in flight) and for this wavefront's
    // fragment reads, meet the others (after which nobody reads the current chunk's stage), refill that stage STAGES
    // chunks ahead, read the next chunk's fragments, then run the current chunk's MFMAs on the fragments read one
    // step earlier; after a tile's last chunk, its epilogue.
    int c = 0, tk = 0;
    auto step = [&](const u32x4 (&xa)[TM], const u32x4 (&xb)[TN], u32x4 (&ya)[TM], u32x4 (&yb)[TN]) {
        meet<LOADS * (STAGES - 2)>();
        issue();
        read_frags(ya, yb);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int t = 0; t < TN; ++t) acc[i][t] = KBlock<T>::mma(xb[t], xa[i], acc[i][t]);
#pragma unroll
        for (int q = 0; q < TM + TN; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
        }
#pragma unroll
        for (int q = 0; q < LOADS; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // vector memory read (the LDS load)
        }
        sched_fence();
        if (++c == nc) {
            epilogue(tk++);
            c = 0;
        }
    };
#pragma unroll
    for (int s = 0; s < STAGES; ++s) issue();
    meet<LOADS * (STAGES - 1)>();
    u32x4 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
    read_frags(fa0, fb0);
    const int steps = my_tiles * nc;  // even: nc is
    for (int g = 0; g < steps; g += 2) {
        step(fa0, fb0, fa1, fb1);
        step(fa1, fb1, fa0, fb0);
    }
    // every wavefront's direct-to-LDS loads land before the workgroup's LDS is released
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
}

template <typename T, int STAGES>
int go_dma_persistent(GemmParams p, hipStream_t stream) {
    constexpr size_t lds = static_cast<size_t>(STAGES) * 512 * 64;
    static std::atomic<uint64_t> done{0};
    const hipError_t attr = allow_dynamic_lds(reinterpret_cast<const void*>(gemm_dma_persistent_kernel<T, STAGES>),
                                              static_cast<int>(lds), done);
    if (attr != hipSuccess) return set_error(-3, "value_proj: LDS size attribute refused: %s", hipGetErrorString(attr));
    p.mt = (p.M + 255) / 256;
    p.nt = (p.NO + 255) / 256;
    const int64_t tiles = static_cast<int64_t>(p.mt) * p.nt;
    p.per_xcd = static_cast<int>((tiles + kXcds - 1) / kXcds);
    // workgroups per XCD: one per CU, a multiple of the channel-tile count, no more than the XCD has tiles for
    int g = (cu_count() / kXcds) / p.nt * p.nt;
    const int need = (p.per_xcd + p.nt - 1) / p.nt * p.nt;
    g = g < need ? g : need;
    if (g <= 0) return go_dma<T, 2, 3>(p, stream);  // more channel tiles than an XCD has CUs
    hipLaunchKernelGGL((gemm_dma_persistent_kernel<T, STAGES>), dim3(g * kXcds), dim3(512), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "value_proj launch failed: %s", hipGetErrorString(e));
}

// variants (td_gemm.hip lists them with the others): 14 = 256 x 128 tiles of 4 wavefronts, one tile per workgroup;
// 18 = the persistent 256 x 256 form; three LDS stages
template <typename T>
int launch_dma_t(GemmParams p, hipStream_t stream, int variant) {
    switch (variant) {
        case 14: return go_dma<T, 2, 3>(p, stream);
        case 18: return go_dma_persistent<T, 3>(p, stream);
        default: return set_error(-1, "value_proj: unknown tile variant %d", variant);
    }
}

// Short, wide projections with float32 output, two weight matrices in one launch (the layer's query prologue: the
// sampling offsets and the attention logits of B * Q query rows): C_j[M, NO_j] = X . W_j^T (+ X2 . W_j^T) + b_j for
// j = 0, 1, float32 accumulation, stored unrounded. With few rows (600 at C = 1024) a tile's share of the operands
// bounds the time, since a CU receives at most about 72 GB/s from L2; so the tiles are small enough for every CU
// to hold one (64 rows x 128 columns; 4 wavefronts of 32 x 64), and both products share one grid.
//
// K streams through a ring of STAGES LDS buffers, STAGES - 1 chunks of 32 ahead, by direct global-to-LDS loads,
// waited for by meet() and laid out with the slot swizzle of gemm_dma_kernel. The product is formed transposed
// (W rows as the MFMA's rows, X rows as its columns), so a lane ends with four consecutive columns of one row: one
// 16-byte store, no LDS pass. The two-operand form adds X2 . W^T by a second MFMA on the same W fragment, so X + X2
// is never rounded. Tiles are numbered column block after column block, C_0's first: the row blocks of a column
// block sit on one XCD and share its W rows in L2.
struct PairParams {
    const void* x;
    const void* x2;
    const void* w[2];
    const void* bias[2];
    float* c[2];
    int M, K, no[2];
    int mt, nt0, tiles, per_xcd;  // 64-row blocks, 128-column blocks of C_0, tiles of both products
    LayerArgs la;                 // FIN: the layer (reference points) and its geometry
    Geom g;
};

// FIN (the layer prologue, L * P a power of two from 4 to 64): the epilogue also does what layer_finalize_kernel
// would do afterwards. C_0's columns 2s, 2s + 1 are sample s's offsets, turned into its location; C_1's are the
// logits, turned into softmax weights over each head's L * P columns, all of which a tile holds: a wavefront's 64
// columns of a row sit in the four lanes that share the row (lane groups kg = 0..3, 16 each), so a head's maximum
// and sum take in-lane steps and at most two cross-lane ones.
template <typename T, int STAGES, bool DUAL, bool FIN>
__global__ __launch_bounds__(256) void gemm_pair_kernel(PairParams p) {
    constexpr int KC = 32, ROW = 64, BM = 64, BN = 128, NA = DUAL ? 2 : 1;
    constexpr int TW = 4, TX = 2;  // 16-row blocks per wavefront: of W (its 64 columns), of each X (its 32 rows)
    constexpr int X_BYTES = BM * ROW, STAGE_BYTES = (NA * BM + BN) * ROW;
    constexpr int LOADS = NA + 2;  // 1 KB wavefront loads per chunk: one 16-row block of each X, two of W
    static_assert(LOADS * (STAGES - 1) <= 63 && STAGES >= 2, "vmcnt range");
    extern __shared__ __align__(16) unsigned char lds[];

    const int unit = static_cast<int>(blockIdx.x % kXcds) * p.per_xcd + static_cast<int>(blockIdx.x / kXcds);
    if (unit >= p.tiles) return;
    const int cb = unit / p.mt, mb = unit - cb * p.mt;
    const int j = cb < p.nt0 ? 0 : 1;
    const int n0 = (j == 0 ? cb : cb - p.nt0) * BN, m0 = mb * BM;
    const int M = p.M, K = p.K, NO = p.no[j];
    const T* __restrict__ X = static_cast<const T*>(p.x);
    const T* __restrict__ X2 = static_cast<const T*>(p.x2);
    const T* __restrict__ W = static_cast<const T*>(p.w[j]);
    const T* __restrict__ bias = static_cast<const T*>(p.bias[j]);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r16 = lane & 15, kg = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;  // the wavefront's rows 32 wm .. + 32 and columns 64 wn .. + 64

    // the bias of the lane's columns, requested first and kept raw until the end (NO % 4 == 0 and an 8-byte
    // aligned bias: four columns are one 8-byte load, and a column block passes NO only by whole quads)
    uint2 braw[TW];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int n = n0 + wn * 64 + t * 16 + 4 * kg;
        braw[t] = uint2{0u, 0u};
        if (bias != nullptr && n < NO) braw[t] = *reinterpret_cast<const uint2*>(bias + n);
    }

    // load sources: wavefront w fills row block w of each X operand and row blocks 2w, 2w + 1 of W; lane =
    // 4 * (row % 16) + slot, the slot holding piece slot ^ g(row). Rows past M or NO load the last valid row.
    const int piece = ((lane & 3) ^ swz(lane >> 2)) * 8;
    int xm = m0 + wave * 16 + (lane >> 2);
    xm = xm < M ? xm : M - 1;
    const T* xs = X + static_cast<size_t>(xm) * K + piece;
    const T* xs2 = DUAL ? X2 + static_cast<size_t>(xm) * K + piece : xs;
    const T* ws[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int n = n0 + (2 * wave + i) * 16 + (lane >> 2);
        n = n < NO ? n : NO - 1;
        ws[i] = W + static_cast<size_t>(n) * K + piece;
    }
    const int nc = K / KC;
    // one group of loads per step, always: past the last chunk the group re-loads it into a stage that is not
    // read for the product again, so every wait is the same constant
    auto issue = [&](int c) {
        unsigned char* st = lds + (c % STAGES) * STAGE_BYTES;
        const int k = (c < nc ? c : nc - 1) * KC;
        load_lds16(xs + k, st + wave * 1024);
        if constexpr (DUAL) load_lds16(xs2 + k, st + X_BYTES + wave * 1024);
        load_lds16(ws[0] + k, st + NA * X_BYTES + 2 * wave * 1024);
        load_lds16(ws[1] + k, st + NA * X_BYTES + (2 * wave + 1) * 1024);
    };

    f32x4 acc[TW][TX];
#pragma unroll
    for (int t = 0; t < TW; ++t)
#pragma unroll
        for (int i = 0; i < TX; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int frag = r16 * ROW + ((kg ^ swz(r16)) << 4);
    const int w_off = NA * X_BYTES + wn * 64 * ROW + frag, x_off = wm * 32 * ROW + frag;
    auto read_frags = [&](int c, u32x4 (&fw)[TW], u32x4 (&fx)[NA][TX]) {
        const unsigned char* st = lds + (c % STAGES) * STAGE_BYTES;
#pragma unroll
        for (int t = 0; t < TW; ++t) fw[t] = *reinterpret_cast<const u32x4*>(st + w_off + t * 16 * ROW);
#pragma unroll
        for (int a = 0; a < NA; ++a)
#pragma unroll
            for (int i = 0; i < TX; ++i)
                fx[a][i] = *reinterpret_cast<const u32x4*>(st + x_off + a * X_BYTES + i * 16 * ROW);
    };
    // step c: wait for chunk c + 1 and meet (nobody reads chunk c's stage any more), refill that stage with chunk
    // c + STAGES, read chunk c + 1's fragments, run chunk c's MFMAs on the fragments read one step earlier
    auto step = [&](int c, const u32x4 (&fw)[TW], const u32x4 (&fx)[NA][TX], u32x4 (&gw)[TW], u32x4 (&gx)[NA][TX]) {
        meet<LOADS * (STAGES - 2)>();
        issue(c + STAGES);
        read_frags(c + 1, gw, gx);
#pragma unroll
        for (int a = 0; a < NA; ++a)  // operand outermost: consecutive MFMAs write different accumulators
#pragma unroll
            for (int t = 0; t < TW; ++t)
#pragma unroll
                for (int i = 0; i < TX; ++i) acc[t][i] = KBlock<T>::mma(fw[t], fx[a][i], acc[t][i]);
        if constexpr (DUAL) {  // spread the next chunk's reads and loads over the 16 MFMAs
#pragma unroll
            for (int r = 0; r < TW + NA * TX; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // LDS read
            }
#pragma unroll
            for (int r = 0; r < LOADS; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // vector memory read (the LDS load)
            }
        }
        sched_fence();
    };
#pragma unroll
    for (int c = 0; c < STAGES; ++c) issue(c);
    meet<LOADS * (STAGES - 1)>();
    u32x4 fw0[TW], fx0[NA][TX], fw1[TW], fx1[NA][TX];
    read_frags(0, fw0, fx0);
    for (int c = 0; c < nc; c += 2) {  // nc is even
        step(c, fw0, fx0, fw1, fx1);
        step(c + 1, fw1, fx1, fw0, fx0);
    }
    meet<0>();  // the tail's re-loads have landed before the workgroup ends

    float* __restrict__ C = p.c[j];
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const T* bt = reinterpret_cast<const T*>(&braw[t]);
        const f32x4 bv = {cvt<float>(bt[0]), cvt<float>(bt[1]), cvt<float>(bt[2]), cvt<float>(bt[3])};
#pragma unroll
        for (int i = 0; i < TX; ++i) acc[t][i] += bv;
    }
    if constexpr (FIN) {
        const Geom& g = p.g;
        const int LP = g.LP;
        if (j == 0) {
#pragma unroll
            for (int t = 0; t < TW; ++t) {
                const int n = n0 + wn * 64 + t * 16 + 4 * kg;
                if (n >= NO) continue;
                // samples s0 and s0 + 1 of a head (n is a multiple of 4, so both are the same head's)
                const int s0 = (n >> 1) & (LP - 1), l0 = s0 / g.P, l1 = (s0 + 1) / g.P;
#pragma unroll
                for (int i = 0; i < TX; ++i) {
                    const int m = m0 + wm * 32 + i * 16 + r16;
                    if (m >= M) continue;
                    const int b = m / g.Q, q = m - b * g.Q;
                    const f32x4 v = acc[t][i];
                    float x0, y0, x1, y1;
                    layer_location<T, float>(p.la, g, b, q, l0, v[0], v[1], x0, y0);
                    layer_location<T, float>(p.la, g, b, q, l1, v[2], v[3], x1, y1);
                    *reinterpret_cast<f32x4*>(C + static_cast<size_t>(m) * NO + n) = f32x4{x0, y0, x1, y1};
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < TX; ++i) {
                // the lane's columns are t * 16 + 4 kg + e of its wavefront's 64; a head's LP columns share
                // t >> log2(LP / 16) and kg >> log2(LP / 4). Every lane takes part in the cross-lane steps, valid
                // or not (columns past NO form whole heads of their own).
                float mx[TW], sm[TW];
#pragma unroll
                for (int t = 0; t < TW; ++t) {
                    const f32x4 v = acc[t][i];
                    mx[t] = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
                    if (LP >= 8) mx[t] = fmaxf(mx[t], xor_lane(mx[t], 16));
                    if (LP >= 16) mx[t] = fmaxf(mx[t], xor_lane(mx[t], 32));
                }
                if (LP >= 32) {
                    mx[0] = mx[1] = fmaxf(mx[0], mx[1]);
                    mx[2] = mx[3] = fmaxf(mx[2], mx[3]);
                }
                if (LP >= 64) mx[0] = mx[1] = mx[2] = mx[3] = fmaxf(mx[0], mx[2]);
#pragma unroll
                for (int t = 0; t < TW; ++t) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[t][i][e] = exp_acc(acc[t][i][e] - mx[t]);
                    const f32x4 v = acc[t][i];
                    sm[t] = (v[0] + v[1]) + (v[2] + v[3]);
                    if (LP >= 8) sm[t] += xor_lane(sm[t], 16);
                    if (LP >= 16) sm[t] += xor_lane(sm[t], 32);
                }
                if (LP >= 32) {
                    sm[0] = sm[1] = sm[0] + sm[1];
                    sm[2] = sm[3] = sm[2] + sm[3];
                }
                if (LP >= 64) sm[0] = sm[1] = sm[2] = sm[3] = sm[0] + sm[2];
                const int m = m0 + wm * 32 + i * 16 + r16;
#pragma unroll
                for (int t = 0; t < TW; ++t) {
                    const int n = n0 + wn * 64 + t * 16 + 4 * kg;
                    if (m < M && n < NO)
                        *reinterpret_cast<f32x4*>(C + static_cast<size_t>(m) * NO + n) = acc[t][i] * (1.f / sm[t]);
                }
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < TW; ++t) {
        const int n = n0 + wn * 64 + t * 16 + 4 * kg;
        if (n >= NO) continue;
#pragma unroll
        for (int i = 0; i < TX; ++i) {
            const int m = m0 + wm * 32 + i * 16 + r16;
            if (m < M) *reinterpret_cast<f32x4*>(C + static_cast<size_t>(m) * NO + n) = acc[t][i];
        }
    }
}

template <typename T, int STAGES, bool DUAL, bool FIN>
int go_pair(PairParams p, hipStream_t stream) {
    constexpr size_t lds = static_cast<size_t>(STAGES) * ((DUAL ? 2 : 1) * 64 + 128) * 64;
    static_assert(lds <= 65536, "within the default dynamic LDS limit");
    p.per_xcd = (p.tiles + kXcds - 1) / kXcds;
    hipLaunchKernelGGL((gemm_pair_kernel<T, STAGES, DUAL, FIN>), dim3(static_cast<unsigned>(p.per_xcd * kXcds)),
                       dim3(256), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "layer prologue launch failed: %s", hipGetErrorString(e));
}

// 4 stages (64 KB with two operands): C = 1024, 600 rows, 3072 columns in 240 tiles: 20.0 µs for the prologue with
// a separate finalize, against 21.3 with 8 stages and 45.9 for two launches of 64 x 64 register-operand tiles
// (graph-timed).
template <typename T, bool FIN>
int launch_pair_t(const PairParams& p, hipStream_t stream) {
    return p.x2 != nullptr ? go_pair<T, 4, true, FIN>(p, stream) : go_pair<T, 4, false, FIN>(p, stream);
}

}  // namespace

int launch_proj_f32_pair(int dtype, const void* x, const void* x2, const void* w0, const void* b0, float* c0,
                         int64_t no0, const void* w1, const void* b1, float* c1, int64_t no1, int64_t M, int64_t K,
                         hipStream_t stream, const LayerArgs* fin, const Geom* g) {
    const uintptr_t a16 = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(x2) |
                          reinterpret_cast<uintptr_t>(w0) | reinterpret_cast<uintptr_t>(w1) |
                          reinterpret_cast<uintptr_t>(c0) | reinterpret_cast<uintptr_t>(c1);
    const uintptr_t a8 = reinterpret_cast<uintptr_t>(b0) | reinterpret_cast<uintptr_t>(b1);
    const int64_t lim = int64_t{1} << 31;
    if ((dtype != kF16 && dtype != kBF16) || a16 % 16 != 0 || a8 % 8 != 0 || K <= 0 || K % 64 != 0 || M <= 0 ||
        no0 <= 0 || no1 <= 0 || no0 % 4 != 0 || no1 % 4 != 0 || M * K >= lim || no0 * K >= lim || no1 * K >= lim ||
        M * no0 >= lim || M * no1 >= lim)
        return 1;
    PairParams p{x, x2, {w0, w1}, {b0, b1}, {c0, c1}, static_cast<int>(M), static_cast<int>(K),
                 {static_cast<int>(no0), static_cast<int>(no1)}, 0, 0, 0, 0, LayerArgs{}, Geom{}};
    p.mt = static_cast<int>((M + 63) / 64);
    p.nt0 = static_cast<int>((no0 + 127) / 128);
    const int64_t tiles = static_cast<int64_t>(p.mt) * (p.nt0 + (no1 + 127) / 128);
    if (tiles >= lim / kXcds) return 1;
    p.tiles = static_cast<int>(tiles);
    const int LP = g != nullptr ? g->LP : 0;
    if (fin != nullptr && g != nullptr && g->P > 0 && LP >= 4 && LP <= 64 && (LP & (LP - 1)) == 0 &&
        no1 == static_cast<int64_t>(g->H) * LP && no0 == 2 * no1 && M == static_cast<int64_t>(g->B) * g->Q) {
        p.la = *fin;
        p.g = *g;
        const int rc = dtype == kF16 ? launch_pair_t<f16, true>(p, stream) : launch_pair_t<bf16, true>(p, stream);
        return rc == 0 ? 2 : rc;
    }
    return dtype == kF16 ? launch_pair_t<f16, false>(p, stream) : launch_pair_t<bf16, false>(p, stream);
}

bool gemm_persistent_fits(int dtype, const GemmParams& p) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w) |
                         reinterpret_cast<uintptr_t>(p.c) | reinterpret_cast<uintptr_t>(p.bias);
    const int64_t lim = int64_t{1} << 31;
    return (dtype == kF16 || dtype == kBF16) && p.K % 64 == 0 && p.K > 0 && p.M >= 256 && p.NO >= 256 &&
           p.NO % 16 == 0 && p.NO <= 256 * 32 && al % 16 == 0 && p.hm_D % 16 == 0 &&
           static_cast<int64_t>(p.M) * p.K < lim && static_cast<int64_t>(p.NO) * p.K < lim &&
           static_cast<int64_t>(p.M) * p.NO < lim;
}

int launch_gemm_dma(int dtype, GemmParams p, hipStream_t stream, int variant) {
    if (p.K % 64 != 0 || p.K == 0) return set_error(-1, "value_proj: tile variant %d needs K %% 64 == 0", variant);
    if (variant == 18 && !gemm_persistent_fits(dtype, p))
        return set_error(-1, "value_proj: the persistent tiles do not take this shape");
    switch (dtype) {
        case kF16: return launch_dma_t<f16>(p, stream, variant);
        case kBF16: return launch_dma_t<bf16>(p, stream, variant);
        default: return set_error(-1, "value_proj: tile variant %d needs 16-bit operands", variant);
    }
}

}  // namespace td
