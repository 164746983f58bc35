// Fused mode: gather the sampled memory rows, then project one C-vector per (batch, query, head).
//
// For one row (b, q, h), with s over the L*P*4 bilinear corners inside the map,
//   g      = sum_s w_s * memory[b, t_s, :]                  (C values, float32)
//   out[d] = W[h*D+d, :] . g + bias[h*D+d] * sum_s w_s      (d < D)
// which equals projecting every token first and sampling afterwards, because sampling and the weighted sum
// are linear (reference csrc/ma_deform_fused.cu:6-14, README.md:16-22).
//
// fused_vec_kernel (float / half / bfloat16, C a multiple of 16 bytes, 16-byte aligned memory and weight):
//   workgroup = (b, tile of QT queries, h), or for small problems (h, balanced slice of the B * Q rows of head h:
//            every CU then holds the same number of rows to within one); heads vary fastest across workgroups.
//   phase 1  corner table of the QT rows into LDS (with memory under 2 GB, each corner row's byte offset, so that
//            phase 2 gathers by raw buffer loads and an outside corner's load returns zeros).
//   phase 2  gather: CV*SG lanes per row, lane = (corner group sg, 16-byte channel chunk ch); each lane sums
//            every SG-th corner of its row with float32 FMAs, the SG partial sums meet by cross-lane adds,
//            and g lands in LDS as float32.
//   phase 3  projection on MFMA: out[16 x D] = g[16 x C] . W_h^T, split over jobs of one K slice and every N tile
//            (D <= 32) or of one (N tile, K slice) pair, one job per wavefront. 16-bit types use v_mfma_f32_16x16x32_{f16,bf16} with g split as hi + lo (two
//            16-bit values whose sum carries 22 / 16 significant bits), so rounding g to the MFMA input type
//            costs no accuracy; float32 uses v_mfma_f32_16x16x4_f32.
// fused_generic_kernel: any C, any alignment, float64 (float64 accumulation); scalar loads, VALU projection.
#include <stdio.h>

#include "td_internal.h"
#include "td_prologue.h"

// Phase stamps (built only with TD_PHASE_STAMPS, as libtinydeform_phases.so; never in libtinydeform.so). Every
// instantiation of the operator's vector kernel reads the 100 MHz real-time counter at its phase boundaries into
// registers and, at its end, lane 0 of every wavefront of the first kPhaseWgs workgroups stores its 16 stamps to
// td_phase_stamp_buf[workgroup][wavefront][16] (12 wavefront slots per workgroup), so a launch's timeline costs no
// memory traffic until the wavefront is done. Slots: 11 kernel entry, 0 rows decoded, 1 corner table barrier
// passed, 2 gather done, 3 gather barrier passed, 4 projection set up, 5 job start, 6 first chunk done (the
// one-slice-per-CU 16-bit kernel only), 7 MFMAs done, 8 partial sums stored, 9 projection barrier passed, 10 outputs
// stored; 0 where a wavefront passed no such point (5 and 7 are not stamped in the jobs of one (N tile, K slice)).
// td_phase_stamps() copies the buffer to the host.
#ifdef TD_PHASE_STAMPS
constexpr int kPhaseWgs = 1024;
__device__ unsigned long long td_phase_stamp_buf[kPhaseWgs * 12 * 16];
extern "C" int td_phase_stamps(void* host, int64_t count) {
    if (host == nullptr || count < 0 || count > int64_t{kPhaseWgs} * 12 * 16) return -1;
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(td_phase_stamp_buf), static_cast<size_t>(count) * 8) == hipSuccess
               ? 0 : -1;
}
#define TD_STAMP(i)                                                                     \
    do {                                                                                \
        if constexpr (kStamp) stamps_[i] = __builtin_amdgcn_s_memrealtime();            \
    } while (0)
#define TD_STAMP_FLUSH()                                                                \
    do {                                                                                \
        if constexpr (kStamp) {                                                         \
            if ((threadIdx.x & (kWave - 1)) == 0 && blockIdx.x < kPhaseWgs) {           \
                unsigned long long* d_ = td_phase_stamp_buf + (blockIdx.x * 12 + threadIdx.x / kWave) * 16; \
                for (int i_ = 0; i_ < 16; ++i_) d_[i_] = stamps_[i_];                   \
            }                                                                           \
        }                                                                               \
    } while (0)
#else
#define TD_STAMP(i) \
    do {            \
    } while (0)
#define TD_STAMP_FLUSH() \
    do {                 \
    } while (0)
#endif

namespace td {
namespace {

constexpr int kAllN = 2;  // N tiles a projection job takes at once when it takes them all (D <= 32)

struct FusedParams {
    const void* mem;
    const void* w;
    const void* bias;
    const void* loc;
    const void* attn;
    void* out;
    Geom g;
    int C, QT, SG, KS, qtiles;
    int per_xcd, units;  // work-unit mapping (decode_block)
    LayerArgs lay;       // query prologue (layer kernels only)
    // balanced slices (slices > 0): B * Q = slices * slice_rows + slice_extra rows per head
    int slices = 0, slice_rows = 0, slice_extra = 0;
    int alln = 0;  // projection jobs take every N tile (D <= 64), one K slice each
    // divisions by L * P, P, the lanes of a row (CV * SG), CV, Q and D by multiply-high (exact below 2^31)
    FastDiv d_lp, d_p, d_gs, d_cv, d_q, d_d;
    int buf = 0;    // memory under 2 GB (mem_bytes): corner table of byte offsets, buffer-load gather (gather_sum_buf)
    int mem_bytes = 0;
};

// Workgroup index -> work unit (b, query tile, h) with heads fastest. Workgroups are dealt to the 8 XCDs
// round-robin, so unit = (bid % 8) * per_xcd + bid / 8 gives each XCD a contiguous range of units: with a batch of
// 8 images each XCD's L2 holds one image's memory rows instead of all eight. valid = false for the at most 7
// workgroups past the last unit.
struct BlockRow {
    int b, qt, h;
    bool valid;
};
__device__ __forceinline__ BlockRow decode_block(int bid, int H, int qtiles, int per_xcd, int units) {
    const int unit = (bid % kXcds) * per_xcd + bid / kXcds;
    BlockRow r;
    r.valid = unit < units;
    r.h = unit % H;
    const int rest = unit / H;
    r.qt = rest % qtiles;
    r.b = rest / qtiles;
    return r;
}

// The bfloat16 8-wavefront kernel with 8 loads in flight (query tiles of large problems; the plain corner rule) is held
// to 64 VGPRs, so that four workgroups fit a CU: bf16 B8 Q300 22.9 -> 22.1 µs. (The same limit makes the float16 and
// float32 ones, and the general corner rule's, spill: fp16 B4 Q300 14.8 -> 17.4.)
template <typename T, int WAVES, int NB, bool GENERAL, bool LAYER>
__global__ __launch_bounds__(WAVES* kWave)
__attribute__((amdgpu_waves_per_eu(std::is_same<T, bf16>::value && WAVES == 8 && NB == 8 && !GENERAL && !LAYER ? 8 : 1)))
void fused_vec_kernel(FusedParams p) {
    constexpr int NTH = WAVES * kWave;
#ifdef TD_PHASE_STAMPS
    constexpr bool kStamp = !LAYER && WAVES <= 12;
    [[maybe_unused]] unsigned long long stamps_[16] = {};
#endif
    TD_STAMP(11);
    constexpr int V = 16 / static_cast<int>(sizeof(T));
    const Geom& g = p.g;
    const int C = p.C, QT = p.QT, SG = p.SG, CV = C / V;
    const int LP = g.LP, S = 4 * LP, D = g.D;
    // float pitch of a g row (and, for the layer kernel, of a query row) in LDS: 16-byte aligned, rows offset
    // by 4 banks
    const int GP = (LAYER && p.lay.Cq > C ? p.lay.Cq : C) + 4;
    const int NTILE = (D + 15) >> 4, PW = NTILE * 16;
    const int PP = ((3 * LP + 15) & ~15) + 4;  // pitch of a row of the query projections

    extern __shared__ __align__(16) unsigned char smem[];
    Corner<float>* cw = reinterpret_cast<Corner<float>*>(smem);  // [QT][S]
    // rows whose corner groups span two wavefronts (SG > 1, CV * SG = 128 lanes) keep the two halves' sums apart:
    // g = gs + gs2. (With SG = 1 a row wider than a wavefront is split by channels and needs no second half.)
    const bool two = SG > 1 && CV * SG > kWave;
    float* gs = reinterpret_cast<float*>(cw + QT * S);            // [QT][GP]
    float* gs2 = gs + QT * GP;                                     // [QT][GP] (two wavefronts per row)
    float* wsum = gs2 + (two ? QT * GP : 0);                       // [2][16]
    unsigned* gmax = reinterpret_cast<unsigned*>(wsum + 32);      // [1] float16: largest |g| above 2^15 (bits)
    float* part = wsum + 36;                                      // [KS][16][PW]
    float* pro = part + p.KS * 16 * PW;                           // layer: [16][PP] query projections
    float* rstat = pro + 16 * PP;                                 // layer: [16][2] softmax max, 1 / sum

    const T* __restrict__ mem = static_cast<const T*>(p.mem);
    const T* __restrict__ w = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    const T* __restrict__ loc = static_cast<const T*>(p.loc);
    const T* __restrict__ attn = static_cast<const T*>(p.attn);
    T* __restrict__ out = static_cast<T*>(p.out);

    const int tid = threadIdx.x;
    // the workgroup's rows: nrows consecutive (batch, query) rows from rbase (row index b * Q + q) of head h. Tiles
    // (p.slices = 0): QT queries of one image. Balanced slices (p.slices > 0, not the layer kernel): slice s of the
    // B * Q rows, slice_rows + (s < slice_extra) of them, so that every workgroup holds the same number of rows to
    // within one.
    int h, rbase, nrows, q0 = 0, bimg = 0;
    if (!LAYER && p.slices > 0) {
        const int unit = (blockIdx.x % kXcds) * p.per_xcd + blockIdx.x / kXcds;
        if (unit >= p.units) return;
        h = unit % g.H;
        const int slice = unit / g.H;
        rbase = slice * p.slice_rows + (slice < p.slice_extra ? slice : p.slice_extra);
        nrows = p.slice_rows + (slice < p.slice_extra ? 1 : 0);
    } else {
        const BlockRow br = decode_block(blockIdx.x, g.H, p.qtiles, p.per_xcd, p.units);
        if (!br.valid) return;
        h = br.h;
        bimg = br.b;
        q0 = br.qt * QT;
        rbase = br.b * g.Q + q0;
        nrows = g.Q - q0 < QT ? g.Q - q0 : QT;
    }

    if constexpr (LAYER) {
        // phase 0 (layer): sampling offsets and attention logits of the tile's queries for head h, on MFMA; the
        // query rows are staged in the g rows' LDS, which phase 2 overwrites only after the corner table is built
        stage_queries<T, float, true, NTH>(p.lay, bimg, q0, QT, g.Q, gs, GP);
        __syncthreads();
        prologue_mfma<T, WAVES>(p.lay, h, LP, QT, gs, GP, pro, PP);
        __syncthreads();
        prologue_stats<float, NTH>(LP, QT, pro, PP, rstat);
        __syncthreads();
    }

    // phase 1: corner table (tokens, or with p.buf the rows' byte offsets)
    TD_STAMP(0);
    const int sb = p.buf ? C * static_cast<int>(sizeof(T)) : 0;
    if (tid == 0) *gmax = 0u;
    for (int i = tid; i < QT * LP; i += NTH) {
        const int r = static_cast<int>(fast_div(p.d_lp, static_cast<uint32_t>(i))), j = i - r * LP;
        Corner<float>* c4 = cw + r * S + 4 * j;
        if (r < nrows) {
            const int64_t row = static_cast<int64_t>(rbase + r) * g.H + h;
            if constexpr (LAYER) {
                float lx, ly, a;
                prologue_sample<T, float>(p.lay, g, bimg, q0 + r, h, r, j, pro, PP, rstat, lx, ly, a);
                corners_at<float, GENERAL>(lx, ly, a, static_cast<int>(fast_div(p.d_p, j)), g, row, c4, sb);
            } else if constexpr (GENERAL) {
                corner4<T, float, true>(loc, attn, g, row, j, c4, sb);
            } else {
                corner4<T, float, false>(loc, attn, g, row, j, static_cast<int>(fast_div(p.d_p, j)), c4, sb);
            }
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) c4[k] = Corner<float>{p.buf ? kOutside : -1, 0.f};
        }
    }
    __syncthreads();
    TD_STAMP(1);

    // One workgroup per CU (12 wavefronts, 6 loads in flight: the balanced-slice shapes of 16-bit problems) has
    // registers to spare, so each projection job's first two W_h chunks and the epilogue's bias value are requested
    // here, ahead of the gather's loads: they land while the gather runs instead of after it. (Requested at kernel
    // start instead, with the location loads, every CU asks for its W_h at once and the locations queue behind:
    // slower.) The phase-3 loop and the epilogue of these kernels are written apart from the others' (kPre below),
    // so that the other instantiations compile exactly as before.
    constexpr bool kPre = WAVES == 12 && NB == 6 && !LAYER;
    constexpr int KCH = sizeof(T) == 2 ? 32 : 16;  // K per MFMA chunk of a job
    u32x4 wpre[2][kAllN];
    T bpre = static_cast<T>(0.f);
    if constexpr (kPre) {
        const int pw = tid / kWave, pn16 = tid & 15, pkg = (tid & (kWave - 1)) >> 4;
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int nt = 0; nt < kAllN; ++nt) wpre[c][nt] = u32x4{0u, 0u, 0u, 0u};
        if (p.alln && pw < p.KS) {  // job pw's chunks kb and kb + 1, as phase 3 reads them
            const int nk = (C + KCH - 1) / KCH;
            const int kb = pw * nk / p.KS, ke = (pw + 1) * nk / p.KS;
            const T* wr0 = w + (static_cast<size_t>(h) * D + pn16) * C;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int k = (kb + c) * KCH + pkg * (KCH / 4);
#pragma unroll
                for (int nt = 0; nt < kAllN; ++nt)
                    if (kb + c < ke && k < C && nt < NTILE && nt * 16 + pn16 < D)
                        wpre[c][nt] = *reinterpret_cast<const u32x4*>(wr0 + static_cast<size_t>(nt) * 16 * C + k);
            }
        }
        if (bias != nullptr && tid < QT * D)
            bpre = bias[static_cast<size_t>(h) * D + tid - static_cast<int>(fast_div(p.d_d, tid)) * D];
    }

    // phase 2: gather C-wide rows, float32 accumulation
    const int GS = CV * SG;
    for (int it = tid; it < QT * GS; it += NTH) {
        const int r = static_cast<int>(fast_div(p.d_gs, static_cast<uint32_t>(it))), rem = it - r * GS;
        const int sg = static_cast<int>(fast_div(p.d_cv, static_cast<uint32_t>(rem))), ch = rem - sg * CV;
        const uint32_t bimg_r = r < nrows ? fast_div(p.d_q, static_cast<uint32_t>(rbase + r)) : 0;
        const T* mb = mem + static_cast<size_t>(bimg_r) * g.N * C;
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.f;
        float ws = 0.f;
        if (p.buf)
            gather_sum_buf<T, V, NB>(cw + r * S, S, sg, SG, buffer_of(mem, p.mem_bytes),
                                     (bimg_r * static_cast<uint32_t>(g.N) * C + ch * V) * static_cast<uint32_t>(sizeof(T)),
                                     acc, ws);
        else
            gather_sum<T, V, NB>(cw + r * S, S, sg, SG, mb + ch * V, static_cast<size_t>(C), acc, ws);
        for (int m = CV; m < GS && m < kWave; m <<= 1) {
#pragma unroll
            for (int i = 0; i < V; ++i) acc[i] += xor_lane(acc[i], m);
            ws += xor_lane(ws, m);
        }
        if ((rem & (kWave - 1)) < CV) {  // the first corner group of each wavefront holds its wavefront's sums
            const int half = two && rem >= kWave;
            float* dst = (half ? gs2 : gs) + r * GP + ch * V;
#pragma unroll
            for (int i = 0; i < V; i += 4)
                *reinterpret_cast<f32x4*>(dst + i) = f32x4{acc[i], acc[i + 1], acc[i + 2], acc[i + 3]};
            if (ch == 0) wsum[16 * half + r] = ws;
            if constexpr (std::is_same<T, f16>::value) {
                float m = 0.f;
#pragma unroll
                for (int i = 0; i < V; ++i) m = fmaxf(m, fabsf(acc[i]));
                if (two) m *= 2.f;  // bounds the sum of the two halves
                if (m > 32768.f) atomicMax(gmax, __float_as_uint(m));  // rare: un-normalised weights, huge memory
            }
        }
    }
    TD_STAMP(2);
    __syncthreads();
    TD_STAMP(3);

    // phase 3: out[16 x D] = g[16 x C] . W_h^T on MFMA; job = K slice with every N tile (p.alln), else (N tile, K slice)
    const int wave = tid / kWave, lane = tid & (kWave - 1);
    const int n16 = lane & 15, kg = lane >> 4;
    const bool av = n16 < QT;
    const float* ga = gs + (av ? n16 : 0) * GP;
    // float16 splits g into hi + lo halves of 16 bits, and hi overflows past 65504. When some |g| of the workgroup
    // exceeds 2^15, g is scaled by a power of two sc that brings the largest below 2^14 and the products by 1 / sc
    // (both exact), so the output stays what float32 accumulation gives, as in the reference.
    float sc = 1.f, inv_sc = 1.f;
    if constexpr (std::is_same<T, f16>::value) {
        const float mx = __uint_as_float(*gmax);
        if (mx > 32768.f && mx <= 3.4e38f) {
            int e;
            frexpf(mx, &e);  // mx < 2^e
            sc = ldexpf(1.f, 14 - e);
            inv_sc = ldexpf(1.f, e - 14);
        }
    }
    TD_STAMP(4);
    if (kPre && p.alln) {
        // as the p.alln block below, with the job's first two W_h chunks taken from wpre
        const int nk = (C + KCH - 1) / KCH;
        for (int ks = wave; ks < p.KS; ks += WAVES) {
            const int kb = ks * nk / p.KS, ke = (ks + 1) * nk / p.KS;
            f32x4 acc[kAllN];
            bool dv[kAllN];
#pragma unroll
            for (int nt = 0; nt < kAllN; ++nt) {
                acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                dv[nt] = nt < NTILE && nt * 16 + n16 < D;
            }
            const T* wr0 = w + (static_cast<size_t>(h) * D + n16) * C;
            auto chunk = [&](int kk, const u32x4(&braw)[kAllN]) {
                const int k = kk * KCH + kg * (KCH / 4);
                const bool kv = k < C;
                if constexpr (sizeof(T) == 2) {
                    using M = MfmaOp<T>;
                    using frag = typename M::frag;
                    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
                    if (av && kv) {
                        a0 = *reinterpret_cast<const f32x4*>(ga + k);
                        a1 = *reinterpret_cast<const f32x4*>(ga + k + 4);
                        if (two) {
                            a0 += *reinterpret_cast<const f32x4*>(ga + QT * GP + k);
                            a1 += *reinterpret_cast<const f32x4*>(ga + QT * GP + k + 4);
                        }
                        a0 *= sc;
                        a1 *= sc;
                    }
                    frag hi, lo;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const T x0 = static_cast<T>(a0[i]), x1 = static_cast<T>(a1[i]);
                        hi[i] = x0;
                        hi[4 + i] = x1;
                        lo[i] = static_cast<T>(a0[i] - static_cast<float>(x0));
                        lo[4 + i] = static_cast<T>(a1[i] - static_cast<float>(x1));
                    }
#pragma unroll
                    for (int nt = 0; nt < kAllN; ++nt) {
                        if (nt >= NTILE) break;
                        const frag bf = __builtin_bit_cast(frag, braw[nt]);
                        acc[nt] = M::mma(hi, bf, acc[nt]);
                        acc[nt] = M::mma(lo, bf, acc[nt]);
                    }
                } else {
                    f32x4 aq = {0.f, 0.f, 0.f, 0.f};
                    if (av && kv) {
                        aq = *reinterpret_cast<const f32x4*>(ga + k);
                        if (two) aq += *reinterpret_cast<const f32x4*>(ga + QT * GP + k);
                    }
#pragma unroll
                    for (int nt = 0; nt < kAllN; ++nt) {
                        if (nt >= NTILE) break;
                        const f32x4 bq = __builtin_bit_cast(f32x4, braw[nt]);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[j], bq[j], acc[nt], 0, 0, 0);
                    }
                }
            };
            int kk = kb;
            TD_STAMP(5);
            if (ks == wave) {  // the chunks requested before the gather
                if (kk < ke) chunk(kk++, wpre[0]);
                TD_STAMP(6);
                if (kk < ke) chunk(kk++, wpre[1]);
            }
            for (; kk < ke; ++kk) {
                const int k = kk * KCH + kg * (KCH / 4);
                u32x4 braw[kAllN];
#pragma unroll
                for (int nt = 0; nt < kAllN; ++nt) {
                    braw[nt] = u32x4{0u, 0u, 0u, 0u};
                    if (dv[nt] && k < C)
                        braw[nt] = *reinterpret_cast<const u32x4*>(wr0 + static_cast<size_t>(nt) * 16 * C + k);
                }
                chunk(kk, braw);
            }
            TD_STAMP(7);
            float* pp = part + ks * 16 * PW;
#pragma unroll
            for (int nt = 0; nt < kAllN; ++nt) {
                if (nt >= NTILE) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) pp[(4 * kg + i) * PW + nt * 16 + n16] = acc[nt][i];
            }
        }
    } else if (p.alln) {
        // every N tile in each job (D <= 16 kAllN): job = K slice, and g's chunk is read (and, in 16 bits, split into
        // hi + lo) once for all N tiles
        const int nk = (C + KCH - 1) / KCH;
        for (int ks = wave; ks < p.KS; ks += WAVES) {
            TD_STAMP(5);
            const int kb = ks * nk / p.KS, ke = (ks + 1) * nk / p.KS;
            f32x4 acc[kAllN];
            bool dv[kAllN];
#pragma unroll
            for (int nt = 0; nt < kAllN; ++nt) {
                acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
                dv[nt] = nt < NTILE && nt * 16 + n16 < D;
            }
            // row n16 of N tile nt is W_h row nt * 16 + n16
            const T* wr0 = w + (static_cast<size_t>(h) * D + n16) * C;
            for (int kk = kb; kk < ke; ++kk) {
                const int k = kk * KCH + kg * (KCH / 4);
                const bool kv = k < C;
                u32x4 braw[kAllN];
#pragma unroll
                for (int nt = 0; nt < kAllN; ++nt) {
                    braw[nt] = u32x4{0u, 0u, 0u, 0u};
                    if (dv[nt] && kv) braw[nt] = *reinterpret_cast<const u32x4*>(wr0 + static_cast<size_t>(nt) * 16 * C + k);
                }
                if constexpr (sizeof(T) == 2) {
                    using M = MfmaOp<T>;
                    using frag = typename M::frag;
                    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
                    if (av && kv) {
                        a0 = *reinterpret_cast<const f32x4*>(ga + k);
                        a1 = *reinterpret_cast<const f32x4*>(ga + k + 4);
                        if (two) {
                            a0 += *reinterpret_cast<const f32x4*>(ga + QT * GP + k);
                            a1 += *reinterpret_cast<const f32x4*>(ga + QT * GP + k + 4);
                        }
                        a0 *= sc;
                        a1 *= sc;
                    }
                    frag hi, lo;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const T x0 = static_cast<T>(a0[i]), x1 = static_cast<T>(a1[i]);
                        hi[i] = x0;
                        hi[4 + i] = x1;
                        lo[i] = static_cast<T>(a0[i] - static_cast<float>(x0));
                        lo[4 + i] = static_cast<T>(a1[i] - static_cast<float>(x1));
                    }
#pragma unroll
                    for (int nt = 0; nt < kAllN; ++nt) {
                        if (nt >= NTILE) break;
                        const frag bf = __builtin_bit_cast(frag, braw[nt]);
                        acc[nt] = M::mma(hi, bf, acc[nt]);
                        acc[nt] = M::mma(lo, bf, acc[nt]);
                    }
                } else {
                    f32x4 aq = {0.f, 0.f, 0.f, 0.f};
                    if (av && kv) {
                        aq = *reinterpret_cast<const f32x4*>(ga + k);
                        if (two) aq += *reinterpret_cast<const f32x4*>(ga + QT * GP + k);
                    }
#pragma unroll
                    for (int nt = 0; nt < kAllN; ++nt) {
                        if (nt >= NTILE) break;
                        const f32x4 bq = __builtin_bit_cast(f32x4, braw[nt]);
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[j], bq[j], acc[nt], 0, 0, 0);
                    }
                }
            }
            TD_STAMP(7);
            float* pp = part + ks * 16 * PW;
#pragma unroll
            for (int nt = 0; nt < kAllN; ++nt) {
                if (nt >= NTILE) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) pp[(4 * kg + i) * PW + nt * 16 + n16] = acc[nt][i];
            }
        }
    } else if constexpr (sizeof(T) == 2) {
        using M = MfmaOp<T>;
        using frag = typename M::frag;
        const int nk = (C + 31) >> 5;
        for (int job = wave; job < NTILE * p.KS; job += WAVES) {
            const int nt = job % NTILE, ks = job / NTILE;
            const int kb = ks * nk / p.KS, ke = (ks + 1) * nk / p.KS;
            const int d = nt * 16 + n16;
            const bool dv = d < D;
            const T* wr = w + (static_cast<size_t>(h) * D + (dv ? d : 0)) * C;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
            for (int kk = kb; kk < ke; ++kk) {
                const int k = kk * 32 + kg * 8;
                const bool kv = k < C;
                u32x4 braw = {0u, 0u, 0u, 0u};
                if (dv && kv) braw = *reinterpret_cast<const u32x4*>(wr + k);
                f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
                if (av && kv) {
                    a0 = *reinterpret_cast<const f32x4*>(ga + k);
                    a1 = *reinterpret_cast<const f32x4*>(ga + k + 4);
                    if (two) {
                        a0 += *reinterpret_cast<const f32x4*>(ga + QT * GP + k);
                        a1 += *reinterpret_cast<const f32x4*>(ga + QT * GP + k + 4);
                    }
                    a0 *= sc;
                    a1 *= sc;
                }
                frag hi, lo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const T x0 = static_cast<T>(a0[i]), x1 = static_cast<T>(a1[i]);
                    hi[i] = x0;
                    hi[4 + i] = x1;
                    lo[i] = static_cast<T>(a0[i] - static_cast<float>(x0));
                    lo[4 + i] = static_cast<T>(a1[i] - static_cast<float>(x1));
                }
                const frag bf = __builtin_bit_cast(frag, braw);
                acc = M::mma(hi, bf, acc);
                acc = M::mma(lo, bf, acc);
            }
            float* pp = part + ks * 16 * PW;
#pragma unroll
            for (int i = 0; i < 4; ++i) pp[(4 * kg + i) * PW + nt * 16 + n16] = acc[i];
        }
    } else {
        const int nk = (C + 15) >> 4;
        for (int job = wave; job < NTILE * p.KS; job += WAVES) {
            const int nt = job % NTILE, ks = job / NTILE;
            const int kb = ks * nk / p.KS, ke = (ks + 1) * nk / p.KS;
            const int d = nt * 16 + n16;
            const bool dv = d < D;
            const T* wr = w + (static_cast<size_t>(h) * D + (dv ? d : 0)) * C;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
            for (int kk = kb; kk < ke; ++kk) {
                const int k = kk * 16 + kg * 4;
                const bool kv = k < C;
                f32x4 bq = {0.f, 0.f, 0.f, 0.f}, aq = bq;
                if (dv && kv) bq = *reinterpret_cast<const f32x4*>(wr + k);
                if (av && kv) {
                    aq = *reinterpret_cast<const f32x4*>(ga + k);
                    if (two) aq += *reinterpret_cast<const f32x4*>(ga + QT * GP + k);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[j], bq[j], acc, 0, 0, 0);
            }
            float* pp = part + ks * 16 * PW;
#pragma unroll
            for (int i = 0; i < 4; ++i) pp[(4 * kg + i) * PW + nt * 16 + n16] = acc[i];
        }
    }
    TD_STAMP(8);
    __syncthreads();
    TD_STAMP(9);

    // epilogue: sum the K slices, add bias * sum of in-map weights, round once
    if constexpr (kPre) {
        auto emit = [&](int o, T bv) {
            const int r = static_cast<int>(fast_div(p.d_d, static_cast<uint32_t>(o))), d = o - r * D;
            if (r >= nrows) return;
            float v = part[r * PW + d];
            for (int ks = 1; ks < p.KS; ++ks) v += part[(ks * 16 + r) * PW + d];
            v *= inv_sc;
            if (bias != nullptr) v = fmaf(cvt<float>(bv), two ? wsum[r] + wsum[16 + r] : wsum[r], v);
            out[(static_cast<size_t>(rbase + r) * g.H + h) * D + d] = static_cast<T>(v);
        };
        if (tid < QT * D) emit(tid, bpre);  // the bias value requested before the gather
        for (int o = tid + NTH; o < QT * D; o += NTH)
            emit(o, bias != nullptr
                        ? bias[static_cast<size_t>(h) * D + o - static_cast<int>(fast_div(p.d_d, o)) * D]
                        : static_cast<T>(0.f));
        TD_STAMP(10);
        TD_STAMP_FLUSH();
        return;
    }
    for (int o = tid; o < QT * D; o += NTH) {
        const int r = static_cast<int>(fast_div(p.d_d, static_cast<uint32_t>(o))), d = o - r * D;
        if (r >= nrows) continue;
        float v = part[r * PW + d];
        for (int ks = 1; ks < p.KS; ++ks) v += part[(ks * 16 + r) * PW + d];
        v *= inv_sc;
        if (bias != nullptr)
            v = fmaf(cvt<float>(bias[static_cast<size_t>(h) * D + d]), two ? wsum[r] + wsum[16 + r] : wsum[r], v);
        out[(static_cast<size_t>(rbase + r) * g.H + h) * D + d] = static_cast<T>(v);
    }
    TD_STAMP(10);
    TD_STAMP_FLUSH();
}

template <typename T, int WAVES, bool GENERAL>
__global__ __launch_bounds__(WAVES* kWave) void fused_generic_kernel(FusedParams p) {
    using A = typename AccOf<T>::type;
    constexpr int NTH = WAVES * kWave;
    const Geom& g = p.g;
    const int C = p.C, QT = p.QT;
    const int LP = g.LP, S = 4 * LP, D = g.D;

    extern __shared__ __align__(16) unsigned char smem[];
    Corner<A>* cw = reinterpret_cast<Corner<A>*>(smem);  // [QT][S]
    A* gs = reinterpret_cast<A*>(cw + QT * S);           // [QT][C]
    A* wsum = gs + QT * C;                                // [QT]

    const T* __restrict__ mem = static_cast<const T*>(p.mem);
    const T* __restrict__ w = static_cast<const T*>(p.w);
    const T* __restrict__ bias = static_cast<const T*>(p.bias);
    const T* __restrict__ loc = static_cast<const T*>(p.loc);
    const T* __restrict__ attn = static_cast<const T*>(p.attn);
    T* __restrict__ out = static_cast<T*>(p.out);

    const int tid = threadIdx.x;
    const BlockRow br = decode_block(blockIdx.x, g.H, p.qtiles, p.per_xcd, p.units);
    if (!br.valid) return;
    const int q0 = br.qt * QT;

    for (int i = tid; i < QT * LP; i += NTH) {
        const int r = i / LP, j = i - r * LP, q = q0 + r;
        Corner<A>* c4 = cw + r * S + 4 * j;
        if (q < g.Q) {
            corner4<T, A, GENERAL>(loc, attn, g, (static_cast<int64_t>(br.b) * g.Q + q) * g.H + br.h, j, c4);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) c4[k] = Corner<A>{-1, static_cast<A>(0)};
        }
    }
    __syncthreads();

    for (int r = tid; r < QT; r += NTH) {
        A s = 0;
        for (int k = 0; k < S; ++k) s += cw[r * S + k].w;
        wsum[r] = s;
    }
    const T* mb = mem + static_cast<size_t>(br.b) * g.N * C;
    for (int it = tid; it < QT * C; it += NTH) {
        const int r = it / C, c = it - r * C;
        const Corner<A>* cr = cw + r * S;
        A acc = 0;
#pragma unroll 4
        for (int s = 0; s < S; ++s) {
            const Corner<A> cc = cr[s];
            const T v = mb[static_cast<size_t>(cc.tok < 0 ? 0 : cc.tok) * C + c];
            acc = fma(cc.w, cc.tok < 0 ? static_cast<A>(0) : cvt<A>(v), acc);
        }
        gs[r * C + c] = acc;
    }
    __syncthreads();

    const int wave = tid / kWave, lane = tid & (kWave - 1);
    for (int o = wave; o < QT * D; o += WAVES) {  // o is uniform across the wavefront
        const int r = o / D, d = o - r * D, q = q0 + r;
        if (q >= g.Q) continue;
        const T* wr = w + (static_cast<size_t>(br.h) * D + d) * C;
        A s = 0;
        for (int c = lane; c < C; c += kWave) s = fma(cvt<A>(wr[c]), gs[r * C + c], s);
        s = wave_sum(s);
        if (lane == 0) {
            if (bias != nullptr) s = fma(cvt<A>(bias[static_cast<size_t>(br.h) * D + d]), wsum[r], s);
            out[((static_cast<size_t>(br.b) * g.Q + q) * g.H + br.h) * D + d] = static_cast<T>(s);
        }
    }
}

constexpr size_t kLdsBudget = 65536;
constexpr size_t kGenericLdsBudget = 160 * 1024;  // MI355X: 160 KB of LDS per CU

inline bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

// Sets the work-unit mapping and returns the grid size (a multiple of the XCD count).
inline int64_t map_units(FusedParams& p) {
    const int64_t units = p.slices > 0 ? static_cast<int64_t>(p.slices) * p.g.H
                                       : static_cast<int64_t>(p.g.B) * p.g.H * p.qtiles;
    p.units = static_cast<int>(units);
    p.per_xcd = static_cast<int>((units + kXcds - 1) / kXcds);
    return static_cast<int64_t>(p.per_xcd) * kXcds;
}

template <typename T, int WAVES, bool LAYER, int NB>
int go_vec_nb(FusedParams p, size_t lds, hipStream_t stream) {
    const int64_t blocks = map_units(p);
    if (p.g.general())
        hipLaunchKernelGGL((fused_vec_kernel<T, WAVES, 8, true, LAYER>), dim3(static_cast<unsigned>(blocks)),
                           dim3(WAVES * kWave), lds, stream, p);
    else
        hipLaunchKernelGGL((fused_vec_kernel<T, WAVES, NB, false, LAYER>), dim3(static_cast<unsigned>(blocks)),
                           dim3(WAVES * kWave), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "fused_vec launch failed: %s", hipGetErrorString(e));
}

// nb: corner loads in flight per lane, 8 or 6 (the plain kernel only; 6 keeps it at 64 VGPRs, 8 wavefronts per SIMD)
template <typename T, int WAVES, bool LAYER>
int go_vec(FusedParams p, size_t lds, hipStream_t stream, int nb = 8) {
    if constexpr (!LAYER) {
        if (nb == 6) return go_vec_nb<T, WAVES, LAYER, 6>(p, lds, stream);
    }
    return go_vec_nb<T, WAVES, LAYER, 8>(p, lds, stream);
}

// The generic kernel may take up to the CU's whole LDS (wide float64 rows: C = 8192 needs 68 KB at one row per
// workgroup); launches above 64 KB need the attribute, set once per instantiation and device.
template <auto Kernel>
int allow_lds(size_t lds) {
    if (lds <= 65536) return 0;
    static std::atomic<uint64_t> done{0};
    const hipError_t attr =
        allow_dynamic_lds(reinterpret_cast<const void*>(Kernel), static_cast<int>(kGenericLdsBudget), done);
    return attr == hipSuccess ? 0 : set_error(-3, "fused_generic: LDS size attribute refused: %s", hipGetErrorString(attr));
}

template <typename T, int WAVES>
int go_generic(FusedParams p, size_t lds, hipStream_t stream) {
    const int64_t blocks = map_units(p);
    const int rc = p.g.general() ? allow_lds<fused_generic_kernel<T, WAVES, true>>(lds)
                                 : allow_lds<fused_generic_kernel<T, WAVES, false>>(lds);
    if (rc != 0) return rc;
    if (p.g.general())
        hipLaunchKernelGGL((fused_generic_kernel<T, WAVES, true>), dim3(static_cast<unsigned>(blocks)),
                           dim3(WAVES * kWave), lds, stream, p);
    else
        hipLaunchKernelGGL((fused_generic_kernel<T, WAVES, false>), dim3(static_cast<unsigned>(blocks)),
                           dim3(WAVES * kWave), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "fused_generic launch failed: %s", hipGetErrorString(e));
}

inline bool aligned16(const void* ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; }


// layer: the query prologue runs inside the kernel (LayerArgs in p.lay); returns 1 without launching anything when
// the vector kernel cannot take the problem (alignment, channel counts, LDS), so the caller can fall back to the
// standalone prologue followed by the plain kernels.
template <typename T>
int launch_fused_t(FusedParams p, hipStream_t stream, const FusedTune& tune, bool layer) {
    using A = typename AccOf<T>::type;
    const Geom& g = p.g;
    const int LP = g.LP, S = 4 * LP, C = p.C, D = g.D;
    const int qmax = g.Q < 16 ? g.Q : 16;

    if constexpr (!std::is_same<T, double>::value) {
        constexpr int V = 16 / static_cast<int>(sizeof(T));
        bool aligned = aligned16(p.mem) && aligned16(p.w) && C % V == 0 && C > 0;
        if (layer) {
            const LayerArgs& la = p.lay;
            aligned = aligned && la.Cq > 0 && la.Cq % V == 0 && aligned16(la.query) && aligned16(la.off_w) &&
                      aligned16(la.aw_w) && (la.pos == nullptr || aligned16(la.pos)) && g.P > 0;
        }
        if (aligned && !tune.generic) {
            const int CV = C / V;
            // Launch shape (measured on MI355X): small problems want one row per wavefront and one pass per
            // workgroup (more workgroups in flight); large ones 8-wave workgroups of 16 rows.
            const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
            const bool big = rows >= 8192;
            int waves = tune.waves ? tune.waves : big ? 8 : 4;
            int sg = tune.sg;
            if (sg <= 0) {
                sg = 1;
                if (!big && is_pow2(CV) && CV < kWave) {
                    sg = kWave / CV;
                    while (sg > 1 && S / sg < 4) sg >>= 1;
                }
            }
            // corner groups of one row span at most two wavefronts, and more than one only in whole wavefronts
            if (sg > 1 && !(is_pow2(CV) && is_pow2(sg) && (CV * sg <= kWave || (CV * sg == 2 * kWave && CV <= kWave))))
                sg = 1;
            const int GS = CV * sg;
            // small problems whose rows are wider than a wavefront but do not tile four wavefronts (16-bit C = 768:
            // two rows of 96 lanes leave a quarter of them idle) take 12 wavefronts when whole rows fill them:
            // C = 768, 12 heads, fp16 B1 Q450 60.0 -> 36.9 µs, bf16 B2 Q150 42.9 -> 26.3, fp32 B1 Q300 118 -> 62
            // (large problems keep 8 wavefronts: fp16 B5 Q150 55.4 against 57.0; the layer kernel has 4 or 8)
            if (tune.waves <= 0 && !big && !layer && GS > kWave && (waves * kWave) % GS != 0 &&
                (12 * kWave) % GS == 0)
                waves = 12;
            const int nth = waves * kWave;
            const int rows_per_pass = nth / GS > 0 ? nth / GS : 1;
            int qt = tune.qt;
            if (qt <= 0) {
                qt = big ? 2 * rows_per_pass : rows_per_pass;
                if (!big && qt > 1 && rows / qt < 300) qt /= 2;
            }
            if (qt > qmax) qt = qmax;
            if (qt < 1) qt = 1;
            // Small problems take balanced slices instead of query tiles: slice s of head h holds (batch, query)
            // rows s * slice_rows + min(s, slice_extra) onward, slice_rows + (s < slice_extra) of them, so every CU
            // holds the same number of rows to within one. Shapes measured on MI355X (graph-timed µs, fixed 4-row
            // tiles -> chosen shape):
            //  * when one workgroup per CU takes at most 6 rows, 16-bit rows are gathered by two wavefronts each
            //    (corner groups over 128 lanes, 6 loads in flight per lane): RT-DETR fp16 B1 Q50 6.28 -> 5.74,
            //    Q100 6.73 -> 5.87, Q150 7.03 -> 6.68;
            //  * otherwise one wavefront per row, with k workgroups per CU for the smallest k whose slices fit 12
            //    rows (k <= 2; 12-wavefront workgroups) or 8 rows (8 wavefronts): fp16 B1 Q300 8.94 (tiles) ->
            //    8.66 (two 8-wavefront slices of 4-5 rows per CU) -> 8.18 (one 12-wavefront slice of 9-10 rows),
            //    fp32 B1 Q300 14.02 -> 12.37, fp16 B2 Q300 12.20 -> 11.93, fp16 B3 Q300 (four 8-row slices per CU,
            //    6 loads in flight so that 32 wavefronts fit) 16.50 -> 15.25.
            const int NTILE = (D + 15) / 16;
            const int nk = sizeof(T) == 2 ? (C + 31) / 32 : (C + 15) / 16;
            const int GP = (layer && p.lay.Cq > C ? p.lay.Cq : C) + 4;
            const int PP = ((3 * LP + 15) & ~15) + 4;
            // Projection jobs. D <= 32: each job takes every N tile of one K slice, so g's chunks are read (and in 16 bits
            // split into hi + lo) once instead of once per N tile; 16-bit types use 4 K slices, one job per SIMD, float32
            // one per wavefront. Measured on MI355X against one job per (N tile, K slice) (graph-timed µs): fp16 B1
            // Q300 8.34 -> 8.03, Q50 5.80 -> 5.62, Q100 6.04 -> 5.83, B2 Q300 11.97 -> 11.15, bf16 B1 Q300 8.52 ->
            // 8.20; float32 B1 Q300 12.45 -> 12.37 (4 slices: 12.80). Larger D keeps one job per (N tile, K slice).
            const bool alln = NTILE <= kAllN;
            auto k_slices = [&](int w) {
                int ks = !alln ? w / NTILE : sizeof(T) == 2 ? (w < 4 ? w : 4) : w;
                return ks < 1 ? 1 : ks > nk ? nk : ks;
            };
            // LDS bytes of a workgroup of q rows, w wavefronts, gathered by corner groups sgx
            auto lds_of = [&](int q, int w, int sgx) {
                const size_t halves = sgx > 1 && CV * sgx > kWave ? 2 : 1;
                return static_cast<size_t>(q) * S * sizeof(Corner<float>) + halves * q * GP * 4 + 36 * 4 +
                       static_cast<size_t>(k_slices(w)) * 16 * NTILE * 16 * 4 +
                       (layer ? static_cast<size_t>(16 * PP + 32) * 4 : 0);
            };
            int64_t slices = 0;
            int nb = 8;
            const int64_t BQ = static_cast<int64_t>(g.B) * g.Q;
            if (!layer && !big && GS == kWave && tune.qt <= 0 && tune.waves <= 0 && tune.sg <= 0) {
                const int cus = cu_count();
                auto slices_for = [&](int k) {
                    int64_t sl = static_cast<int64_t>(k) * cus / g.H;
                    return sl < 1 ? int64_t{1} : sl > BQ ? BQ : sl;
                };
                const int64_t s1 = slices_for(1), per1 = (BQ + s1 - 1) / s1;
                int s_qt = 0, s_waves = 0, s_sg = sg, s_nb = 8;
                if (sizeof(T) == 2 && S / (2 * sg) >= 4 && per1 <= 6) {
                    s_sg = 2 * sg;  // CV * s_sg = 128: two whole wavefronts per row
                    slices = s1;
                    s_qt = static_cast<int>(per1);
                    s_waves = 2 * s_qt <= 8 ? 8 : 12;
                    s_nb = 6;
                } else {
                    for (int k = 1; k <= 4 && slices == 0; ++k) {
                        const int64_t sl = slices_for(k), per = (BQ + sl - 1) / sl;
                        if (per <= 8 || (k <= 2 && per <= 12)) {
                            slices = sl;
                            s_qt = static_cast<int>(per);
                            s_waves = per <= 8 ? 8 : 12;
                            // 6 loads in flight where 8 (80 VGPRs: 24 wavefronts per CU) do not fit, and for 16-bit
                            // rows in one 12-wavefront slice per CU (fp16 B1 Q300 8.25 -> 8.18 µs, bf16 8.47 ->
                            // 8.38; two slices per CU or float32 measured faster with 8)
                            s_nb = k * s_waves > 24 || (sizeof(T) == 2 && k == 1 && s_waves == 12) ? 6 : 8;
                        }
                    }
                }
                // a slice's rows must all fit one workgroup's LDS; otherwise query tiles
                if (slices > 0 && lds_of(s_qt, s_waves, s_sg) <= kLdsBudget) {
                    qt = s_qt;
                    waves = s_waves;
                    sg = s_sg;
                    nb = s_nb;
                } else {
                    slices = 0;
                }
            }
            const int ks = k_slices(waves);
            auto lds = [&](int q) { return lds_of(q, waves, sg); };
            while (qt > 1 && lds(qt) > kLdsBudget) --qt;
            if (lds(qt) <= kLdsBudget) {
                p.QT = qt;
                p.SG = sg;
                p.KS = ks;
                if (LP > 0) p.d_lp = make_fastdiv(static_cast<uint32_t>(LP));
                if (g.P > 0) p.d_p = make_fastdiv(static_cast<uint32_t>(g.P));
                p.d_gs = make_fastdiv(static_cast<uint32_t>(CV * sg));
                p.d_cv = make_fastdiv(static_cast<uint32_t>(CV));
                if (g.Q > 0) p.d_q = make_fastdiv(static_cast<uint32_t>(g.Q));
                if (D > 0) p.d_d = make_fastdiv(static_cast<uint32_t>(D));
                const int64_t mem_bytes = static_cast<int64_t>(g.B) * g.N * C * static_cast<int64_t>(sizeof(T));
                p.buf = mem_bytes > 0 && mem_bytes < (int64_t{1} << 31) ? 1 : 0;
                p.mem_bytes = p.buf ? static_cast<int>(mem_bytes) : 0;
                p.alln = alln ? 1 : 0;
                p.qtiles = (g.Q + qt - 1) / qt;
                if (slices > 0) {
                    p.slices = static_cast<int>(slices);
                    p.slice_rows = static_cast<int>(BQ / slices);
                    p.slice_extra = static_cast<int>(BQ % slices);
                }
                if (tune.plan != nullptr) {
                    const int64_t units = slices > 0 ? slices * g.H : static_cast<int64_t>(g.B) * g.H * p.qtiles;
                    const int64_t rows_max = slices > 0 ? p.slice_rows + (p.slice_extra > 0 ? 1 : 0) : qt;
                    *tune.plan = LaunchPlan{{0, units, waves, qt, slices, rows_max, sg, p.g.general() ? 8 : nb}};
                    return 0;
                }
                // corner loads in flight per lane: 8 (6 for the slice shapes above that need it)
                if (layer) {
                    switch (waves) {
                        case 4: return go_vec<T, 4, true>(p, lds(qt), stream);
                        case 8: return go_vec<T, 8, true>(p, lds(qt), stream);
                        default: return set_error(-1, "fused layer: waves must be 4 or 8 (got %d)", waves);
                    }
                }
                switch (waves) {
                    case 4: return go_vec<T, 4, false>(p, lds(qt), stream, nb);
                    case 8: return go_vec<T, 8, false>(p, lds(qt), stream, nb);
                    case 12: return go_vec<T, 12, false>(p, lds(qt), stream, nb);
                    default: return set_error(-1, "fused: waves must be 4, 8 or 12 (got %d)", waves);
                }
            }
        }
    }
    if (layer) return 1;
    // generic kernel
    auto lds = [&](int q) {
        return static_cast<size_t>(q) * S * sizeof(Corner<A>) + static_cast<size_t>(q) * C * sizeof(A) +
               static_cast<size_t>(q) * sizeof(A);
    };
    int qt = tune.qt > 0 ? tune.qt : 4;
    if (qt > qmax) qt = qmax;
    if (qt < 1) qt = 1;
    while (qt > 1 && lds(qt) > kLdsBudget) --qt;
    if (lds(qt) > kGenericLdsBudget)
        return set_error(-1, "channels (%d) too large for the %s fused kernel", C, sizeof(T) == 8 ? "float64" : "scalar");
    p.QT = qt;
    p.SG = 1;
    p.KS = 1;
    p.qtiles = (g.Q + qt - 1) / qt;
    if (tune.plan != nullptr) {
        *tune.plan = LaunchPlan{{1, static_cast<int64_t>(g.B) * g.H * p.qtiles, 4, qt, 0, qt, 1, 1}};
        return 0;
    }
    return go_generic<T, 4>(p, lds(qt), stream);
}

}  // namespace

int launch_fused(int dtype, const void* mem, const void* w, const void* bias, const Geom& g, int C, const void* loc,
                 const void* attn, void* out, hipStream_t stream, const FusedTune& tune, const LayerArgs* layer) {
    FusedParams p{mem, w, bias, loc, attn, out, g, C, 1, 1, 1, 1, 0, 0, LayerArgs{}};
    if (layer != nullptr) p.lay = *layer;
    const bool lay = layer != nullptr;
    switch (dtype) {
        case kF32: return launch_fused_t<float>(p, stream, tune, lay);
        case kF16: return launch_fused_t<f16>(p, stream, tune, lay);
        case kBF16: return launch_fused_t<bf16>(p, stream, tune, lay);
        case kF64: return lay ? 1 : launch_fused_t<double>(p, stream, tune, false);
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
}

}  // namespace td
