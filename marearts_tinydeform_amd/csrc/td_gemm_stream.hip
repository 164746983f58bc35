// Streaming value projection for narrow K: value[M, 256] = memory[M, K] . W[256, K]^T + bias, K = 128 or 256,
// 16-bit operands (the C = 256 projections of RT-DETR, DINO and Deformable-DETR decoders).
//
// At K <= 256 the product is bound by HBM: each token row is read once (K * 2 bytes) and its value row written once
// (512 bytes), 128 flops per byte, below MI355X's ridge. A tiled GEMM spends a tile's short life (K / 32 chunks)
// on staging W and crossing barriers; this kernel keeps W resident and streams the tokens:
//   * one workgroup of four wavefronts per CU (persistent grid), each workgroup an equal share of M;
//   * every wavefront holds a quarter of W (64 output channels x K, 128 VGPRs at K = 256) in registers for the whole
//     kernel. W reaches them through LDS: at kernel start the workgroup's direct global-to-LDS loads bring W in
//     whole 1 KB runs (8 full 128-byte lines per load; a register load of a fragment would touch 16 half lines), into
//     an LDS copy whose 16-byte chunk c of row ch sits at slot ch * (K / 8) + (c ^ key(ch)), key(ch) = the row's
//     position in its 16 x 16 output tile (bits 3-4 and 0-1 of ch), so that each fragment read (16 rows, one chunk
//     each) hits 16 distinct 16-byte bank groups; each wavefront then reads its quarter into registers. With W
//     (128 KB at K = 256) and the two token stages the workgroup holds the CU's whole 160 KB of LDS;
//   * the token rows stream through LDS in steps of 32 tokens: two stages, the next step's rows requested by direct
//     global-to-LDS loads while this step's MFMAs run, and the four wavefronts share each staged row (each computing
//     its 64 channels of it), so a token row is read from memory once per CU;
//   * the product is formed transposed, D = W . tokens^T on v_mfma_f32_16x16x32, so a lane's 4 accumulators are 4
//     output channels of one token. The W rows of the 16 x 16 output tiles are permuted so that tiles 2p and 2p + 1
//     give lane (r, kg) channels 32 p + 8 kg .. + 3 and + 4 .. + 7 of token r: 8 consecutive channels, one 16-byte
//     store (row 4 a + b of tile 2p + h is channel 32 p + 8 a + 4 h + b of the wavefront's quarter).
// Token row j of a step (0..31) sits in its stage as K / 8 chunks of 16 bytes, chunk c at slot c ^ (j & 15): a
// fragment read (16 rows, one chunk each) then hits 16 distinct 16-byte bank groups.
//
// Measured on MI355X against the earlier form of this kernel (W in LDS, each wavefront loading its own tokens into
// registers, graph-timed µs): RT-DETR B2 (16800 x 256) 10.3 -> 9.1, B8 bf16 (67200) 18.7 -> 17.6, DINO B4 (88892)
// 22.5 -> 20.6, DINO encoder B2 (44446) 14.8 -> 14.0, 80000 x 128 14.1 -> 13.6, 177784 x 256 36.3 -> 34.1. Deeper
// rings measured slower at every size (three stages: B8 18.6, four 19.0, six 20.5): more token rows in flight per CU
// did not raise the memory rate, they delayed the first stage. Timestamps per workgroup then showed the start
// dominating: W's register loads (16 half lines each) took 3.8 µs before the first step and held up the second;
// staging W through LDS in whole lines, with the second stage requested at kernel start too: 16800 x 256
// 9.0 -> 7.6, 33600 12.2 -> 10.3, 44446 14.0 -> 12.0, B8 bf16 17.8 -> 15.9, DINO B4 21.3 -> 18.8, 177784 33.7 ->
// 32.8, 44446 x 128 9.9 -> 8.9. Stores that bypass or write through L2 (nontemporal, sc1) measured no faster.
#include "td_gemm.h"

namespace td {
namespace {

constexpr int kStreamNO = 256;   // output columns
constexpr int kStreamWaves = 4;  // wavefronts per workgroup (one per SIMD)
constexpr int kStreamStep = 32;  // tokens per step

template <typename T>
struct Out8 {
    T v[8];
};

// 16 bytes per lane from global memory straight into LDS: lane i's bytes land at dst + 16 i (dst is the
// wavefront's base, the same for every lane)
__device__ __forceinline__ void load_lds16(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
}

// Wait until at most VM vector-memory operations of this wavefront are in flight and its LDS accesses are done, then
// meet the workgroup at a barrier without the fence of __syncthreads (which would drain every outstanding load). The
// s_waitcnt builtin is seen by the compiler's own wait insertion; the empty asm statements with a memory clobber and
// the scheduling barriers keep memory accesses on their side. Encoding (gfx9): vmcnt in bits 3:0 and 15:14, expcnt
// 6:4 (7 = no wait), lgkmcnt 11:8.
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

// WT: W is given as stored by its owner, [K, 256] with the 256 output channels contiguous (C = A . W: the input
// gradient grad_memory = G . value_weight), instead of [256, K]. Its LDS copy then holds K rows of 256 channels in
// order (the same 1 KB direct loads), and each wavefront reads its W quarter into registers once by LDS transpose
// reads (ds_read_b64_tr_b16: within each 16 lanes, lane i receives element i % 4 of the 8-byte pieces lanes i / 4,
// 4 + i / 4, 8 + i / 4 and 12 + i / 4 point at), lane j pointing at k row 8 kg + j / 4 (+ 4) and at the column of
// its fragment layout's channel group j % 4, so that lane r receives the 8 k of the channel the layout gives it.
template <typename T, int KB, bool WT>
__global__ __launch_bounds__(kStreamWaves* kWave) __attribute__((amdgpu_waves_per_eu(1, 1))) void gemm_stream_kernel(
    GemmParams p) {
    constexpr int NTQ = kStreamNO / 16 / kStreamWaves;  // 16-channel tiles per wavefront: 4
    constexpr int CHR = KB * 4;                         // 16-byte chunks per token row
    constexpr int ROWB = CHR * 16;                      // bytes per token row
    constexpr int STEP = kStreamStep;
    constexpr int SHN = STEP / 16;                      // 16-token halves per step
    constexpr int STAGE = STEP * ROWB;                  // 16 KB (K = 256) or 8 KB (K = 128)
    constexpr int DL = STAGE / 1024 / kStreamWaves;     // 1 KB direct loads per wavefront per stage: 4 or 2
    constexpr int NST = SHN * (NTQ / 2);                // stores per wavefront per step
    static_assert(DL >= 1 && CHR >= 16 && CHR % 16 == 0, "stage layout");
    // Waits, in vector-memory operations that may stay in flight (they complete in issue order):
    //  * before step 0 everything requested at kernel start has landed: stages 0 and 1, W and the bias;
    //  * step i >= 1: its stage was requested before step i - 1's stores (at kernel start for step 1, after the
    //    meeting of step i - 1 otherwise), so those stores may stay in flight.
    constexpr int VM_STEADY = NST;
    static_assert(VM_STEADY <= 63, "vmcnt range");
    extern __shared__ __align__(16) unsigned char smem[];

    const T* __restrict__ A = static_cast<const T*>(p.a);
    const T* __restrict__ W = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    T* __restrict__ C = static_cast<T*>(p.c);
    const int M = p.M, K = p.K;
    const int tid = threadIdx.x, lane = tid & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int r = lane & 15, kg = lane >> 4;
    const int lo = static_cast<int>(static_cast<int64_t>(blockIdx.x) * M / gridDim.x);
    const int hi = static_cast<int>(static_cast<int64_t>(blockIdx.x + 1) * M / gridDim.x);
    const int ns = (hi - lo + STEP - 1) / STEP;
    if (ns <= 0) return;  // the whole workgroup (uniform)
    // the channel quarter of this wavefront, rotated by workgroup so that the CUs of an XCD request different parts
    // of W first
    const int qc = 64 * ((wave + static_cast<int>(blockIdx.x / kXcds)) & 3);

    // direct loads of step i's token rows into stage i % 2; steps past the last re-read the last rows into a stage
    // that is never read, so every step issues the same loads and the waits stay exact
    auto issue = [&](int i) {
        const int m0 = lo + STEP * (i < ns ? i : ns - 1);
        unsigned char* st = smem + (i & 1) * STAGE;
#pragma unroll
        for (int j = 0; j < DL; ++j) {
            const int q = (wave * DL + j) * kWave + lane;  // slot of the stage
            const int row = q / CHR, c = q % CHR;
            int m = m0 + row;
            m = m < hi ? m : hi - 1;
            load_lds16(A + static_cast<size_t>(m) * K + (c ^ (row & 15)) * 8, st + (wave * DL + j) * 1024);
        }
    };
    // the first two stages go out ahead of W, so the first 64 tokens do not queue behind it
    issue(0);
    issue(1);

    // this wavefront's W quarter: tile t, K block kb; lane row r of tile t is channel
    // qc + 32 (t / 2) + 8 (r / 4) + 4 (t % 2) + r % 4
    u32x4 wf[NTQ][KB];
    unsigned char* const wl = smem + 2 * STAGE;  // the LDS copy of W
    auto wkey = [](int ch) { return (((ch >> 3) & 3) << 2) | (ch & 3); };
    {
        constexpr int WDL = kStreamNO * CHR / kWave / kStreamWaves;  // 1 KB direct loads per wavefront: CHR
        const int rot = static_cast<int>(blockIdx.x / kXcds) % WDL;
#pragma unroll 4
        for (int jj = 0; jj < WDL; ++jj) {
            const int j = wave * WDL + (jj + rot) % WDL;  // the CUs of an XCD start on different runs
            const int sl = j * kWave + lane;
            if constexpr (WT) {  // slot sl: k row sl / 32, channels (sl % 32) * 8 .. + 7
                load_lds16(W + static_cast<size_t>(sl / (kStreamNO / 8)) * kStreamNO + (sl % (kStreamNO / 8)) * 8,
                           wl + j * 1024);
            } else {
                const int ch = sl / CHR, c = (sl % CHR) ^ wkey(ch);
                load_lds16(W + static_cast<size_t>(ch) * K + c * 8, wl + j * 1024);
            }
        }
    }
    // the bias is loaded unconditionally (W's first row stands in for a missing one) so that the count of loads in
    // flight is the same with and without it
    Out8<T> bv[NTQ / 2];
#pragma unroll
    for (int pp = 0; pp < NTQ / 2; ++pp)
        bv[pp] = __builtin_bit_cast(
            Out8<T>, *reinterpret_cast<const u32x4*>((bias != nullptr ? bias : W) + qc + 32 * pp + 8 * kg));

    // one step: fragments of step i's stage, MFMAs, stores
    auto step = [&](int i) {
        const unsigned char* st = smem + (i & 1) * STAGE;
        u32x4 tf[SHN][KB];
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int sh = 0; sh < SHN; ++sh)
                tf[sh][kb] = *reinterpret_cast<const u32x4*>(st + (sh * 16 + r) * ROWB + (((kb * 4 + kg) ^ r) << 4));
        f32x4 acc[SHN][NTQ];
#pragma unroll
        for (int sh = 0; sh < SHN; ++sh)
#pragma unroll
            for (int t = 0; t < NTQ; ++t) acc[sh][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
            for (int sh = 0; sh < SHN; ++sh)
#pragma unroll
                for (int t = 0; t < NTQ; ++t) acc[sh][t] = KBlock<T>::mma(wf[t][kb], tf[sh][kb], acc[sh][t]);
        // only the last step can be partial, and no wait follows it, so skipped stores never upset the counts
#pragma unroll
        for (int sh = 0; sh < SHN; ++sh) {
            const int m = lo + STEP * i + 16 * sh + r;
            if (m >= hi) continue;
            T* const row = C + out_row(p, m);
#pragma unroll
            for (int pp = 0; pp < NTQ / 2; ++pp) {
                Out8<T> o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float b0 = bias != nullptr ? cvt<float>(bv[pp].v[e]) : 0.f;
                    const float b1 = bias != nullptr ? cvt<float>(bv[pp].v[4 + e]) : 0.f;
                    o.v[e] = static_cast<T>(acc[sh][2 * pp][e] + b0);
                    o.v[4 + e] = static_cast<T>(acc[sh][2 * pp + 1][e] + b1);
                }
                *reinterpret_cast<u32x4*>(row + out_col(p, qc + 32 * pp + 8 * kg)) = __builtin_bit_cast(u32x4, o);
            }
        }
    };
    // Step 0 is peeled off the loop: its MFMAs wait for W block by block, and the loop then has no register loads
    // left for the compiler to wait on (with step 0 inside, its merged count put a full wait after every step's
    // direct loads). A stage is refilled only after every wavefront has passed the barrier of the step that follows
    // its reads.
    meet<0>();  // stages 0 and 1, W and the bias have landed
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int t = 0; t < NTQ; ++t) {
            if constexpr (WT) {
                using v4s = short __attribute__((ext_vector_type(4)));
                using lds_v4s = __attribute__((address_space(3))) v4s;
                const int k = kb * 32 + kg * 8 + (r >> 2);
                const int col = qc + 32 * (t >> 1) + 8 * (r & 3) + 4 * (t & 1);
                const unsigned char* q = wl + (k * kStreamNO + col) * 2;
                const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(q));
                const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(q + 4 * kStreamNO * 2));
                wf[t][kb] = __builtin_bit_cast(u32x4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            } else {
                const int ch = qc + 32 * (t >> 1) + 8 * (r >> 2) + 4 * (t & 1) + (r & 3);
                wf[t][kb] = *reinterpret_cast<const u32x4*>(wl + (ch * CHR + ((kb * 4 + kg) ^ wkey(ch))) * 16);
            }
        }
    step(0);
    for (int i = 1; i < ns; ++i) {
        meet<VM_STEADY>();
        issue(i + 1);
        step(i);
    }
    // the last refill (never read) lands before the workgroup ends, so no direct load writes LDS that the next
    // workgroup on this CU may own
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0)
}

template <typename T, int KB, bool WT>
int go_stream(GemmParams p, int64_t grid, hipStream_t stream) {
    // two token stages and W: 160 KB at K = 256, 80 KB at K = 128
    constexpr size_t lds = static_cast<size_t>(2) * kStreamStep * KB * 64 + static_cast<size_t>(kStreamNO) * KB * 64;
    if constexpr (lds > 65536) {
        static std::atomic<uint64_t> done{0};
        const hipError_t attr =
            allow_dynamic_lds(reinterpret_cast<const void*>(gemm_stream_kernel<T, KB, WT>), static_cast<int>(lds), done);
        if (attr != hipSuccess)
            return set_error(-3, "value_proj: LDS size attribute refused: %s", hipGetErrorString(attr));
    }
    hipLaunchKernelGGL((gemm_stream_kernel<T, KB, WT>), dim3(static_cast<unsigned>(grid)), dim3(kStreamWaves * kWave), lds,
                       stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "value_proj launch failed: %s", hipGetErrorString(e));
}

// One workgroup per CU (at least one step of tokens each); the workgroups' shares differ by at most one token.
template <typename T, bool WT>
int stream_t(GemmParams p, hipStream_t stream) {
    int64_t grid = (static_cast<int64_t>(p.M) + kStreamStep - 1) / kStreamStep;
    const int cus = cu_count();
    if (grid > cus) grid = cus;
    if (grid < 1) grid = 1;
    return p.K == 256 ? go_stream<T, 8, WT>(p, grid, stream) : go_stream<T, 4, WT>(p, grid, stream);
}

}  // namespace

// The bias is read with 16-byte loads, so it must be 16-byte aligned like the other operands.
bool gemm_stream_fits(int dtype, const GemmParams& p) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(p.a) | reinterpret_cast<uintptr_t>(p.w) |
                         reinterpret_cast<uintptr_t>(p.c) | reinterpret_cast<uintptr_t>(p.bias);
    return (dtype == kF16 || dtype == kBF16) && p.NO == kStreamNO && (p.K == 128 || p.K == 256) && p.M > 0 &&
           al % 16 == 0 && p.hm_D % 8 == 0;
}

int launch_gemm_stream(int dtype, GemmParams p, hipStream_t stream, bool w_stored) {
    if (!gemm_stream_fits(dtype, p)) return set_error(-1, "value_proj: the streaming kernel does not take this shape");
    if (w_stored) return dtype == kF16 ? stream_t<f16, true>(p, stream) : stream_t<bf16, true>(p, stream);
    return dtype == kF16 ? stream_t<f16, false>(p, stream) : stream_t<bf16, false>(p, stream);
}

}  // namespace td
