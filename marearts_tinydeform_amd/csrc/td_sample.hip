// Project mode, second half: sample projected values.
//   out[b, q, h*D + d] = sum_s w_s * value[b, t_s, h*D + d]
// over the L*P*4 bilinear corners of row (b, q, h) that lie inside the map (same corner rule as fused mode).
//
// Rows (b, q, h) are independent and need no shared weights, so a workgroup takes RB consecutive rows.
// Each row is served by DV*SG lanes: lane = (corner group sg, chunk ch of V elements), so one load
// instruction of a wavefront fetches 64 / (DV*SG) * SG rows' D-wide corner rows at once; the SG partial sums
// of a row meet by cross-lane adds (lanes DV, 2*DV, ... apart) and the row is stored with V-element stores.
// With a value tensor under 2 GB the corner table holds byte offsets and the rows come by raw buffer loads
// (gather_sum_buf), an outside corner's load returning zeros.
#include "td_internal.h"

namespace td {
namespace {

struct SampleParams {
    const void* value;
    const void* loc;
    const void* attn;
    void* out;
    Geom g;
    int RB, SG;
    int64_t rows;
    int per_xcd, blocks;  // workgroup -> row-block mapping: XCD x takes a contiguous range of row blocks
    int hq = 0;           // rows taken in (b, h, q) order instead of the (b, q, h) of the output
    // Index arithmetic by multiply-high (exact below 2^31): divisions by LP, P, DV * SG, DV, and with fast
    // (B * Q * H < 2^31) by H, Q and Q * H, instead of the 64-bit division routine (the kernel is issue-bound)
    FastDiv d_lp, d_p, d_gs, d_dv, d_h, d_q, d_qh;
    int fast = 0;
    int buf = 0;    // value under 2 GB (val_bytes): corner table of byte offsets, buffer-load gather (gather_sum_buf)
    int val_bytes = 0;
};

// Row (b, q, h) of the i-th row in the order the workgroups take them: the output's own order, or with hq (b, h, q),
// so that the workgroups of an XCD work through one head's values at a time
__device__ __forceinline__ int64_t sample_row(const SampleParams& p, int64_t i) {
    if (!p.hq) return i;
    if (p.fast) {
        const uint32_t n = static_cast<uint32_t>(i), b = fast_div(p.d_qh, n), rem = n - b * p.g.H * p.g.Q;
        const uint32_t h = fast_div(p.d_q, rem), q = rem - h * p.g.Q;
        return (static_cast<int64_t>(b) * p.g.Q + q) * p.g.H + h;
    }
    const int64_t HQ = static_cast<int64_t>(p.g.H) * p.g.Q;
    const int64_t b = i / HQ, rem = i - b * HQ;
    const int64_t h = rem / p.g.Q, q = rem - h * p.g.Q;
    return (b * p.g.Q + q) * p.g.H + h;
}

template <typename T, int V, int WAVES, int NB, bool GENERAL>
__global__ __launch_bounds__(WAVES* kWave) void sample_kernel(SampleParams p) {
    constexpr int NTH = WAVES * kWave;
    using IO = VecIO<T, V>;
    const Geom& g = p.g;
    const int LP = g.LP, S = 4 * LP, D = g.D, HD = g.H * D;
    const int DV = D / V, SG = p.SG, GS = DV * SG, RB = p.RB;
    extern __shared__ __align__(16) unsigned char smem[];
    Corner<float>* cw = reinterpret_cast<Corner<float>*>(smem);  // [RB][S]

    const T* __restrict__ value = static_cast<const T*>(p.value);
    const T* __restrict__ loc = static_cast<const T*>(p.loc);
    const T* __restrict__ attn = static_cast<const T*>(p.attn);
    T* __restrict__ out = static_cast<T*>(p.out);

    const int tid = threadIdx.x;
    const int rblock = (blockIdx.x % kXcds) * p.per_xcd + blockIdx.x / kXcds;
    if (rblock >= p.blocks) return;
    const int64_t row0 = static_cast<int64_t>(rblock) * RB;

    // corner table: tokens, or with p.buf the rows' byte offsets
    const int sb = p.buf ? (g.value_hm ? D : HD) * static_cast<int>(sizeof(T)) : 0;
    for (int i = tid; i < RB * LP; i += NTH) {
        const int r = static_cast<int>(fast_div(p.d_lp, static_cast<uint32_t>(i))), j = i - r * LP;
        Corner<float>* c4 = cw + r * S + 4 * j;
        if (row0 + r < p.rows) {
            const int64_t row = sample_row(p, row0 + r);
            if constexpr (GENERAL)
                corner4<T, float, true>(loc, attn, g, row, j, c4, sb);
            else
                corner4<T, float, false>(loc, attn, g, row, j, static_cast<int>(fast_div(p.d_p, j)), c4, sb);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) c4[k] = Corner<float>{p.buf ? kOutside : -1, 0.f};
        }
    }
    __syncthreads();

    const int64_t QH = static_cast<int64_t>(g.Q) * g.H;
    for (int it = tid; it < RB * GS; it += NTH) {
        const int r = static_cast<int>(fast_div(p.d_gs, static_cast<uint32_t>(it))), rem = it - r * GS;
        const int sg = static_cast<int>(fast_div(p.d_dv, static_cast<uint32_t>(rem))), ch = rem - sg * DV;
        const bool valid = row0 + r < p.rows;
        const int64_t row = valid ? sample_row(p, row0 + r) : 0;
        int64_t b;
        int h;
        if (p.fast) {  // row = (b * Q + q) * H + h
            const uint32_t rw = static_cast<uint32_t>(row), bq = fast_div(p.d_h, rw);
            h = static_cast<int>(rw - bq * g.H);
            b = fast_div(p.d_q, bq);
        } else {
            b = row / QH;
            h = static_cast<int>(row % g.H);
        }
        // token-major value [B, N, H*D]: head rows HD apart; head-major [B, H, N, D]: D apart, so a bilinear pair
        // (x0, x0 + 1) is one contiguous 2 D-element run
        const T* base = g.value_hm ? value + (static_cast<size_t>(b) * g.H + h) * g.N * D + ch * V
                                   : value + static_cast<size_t>(b) * g.N * HD + static_cast<size_t>(h) * D + ch * V;
        const size_t stride = g.value_hm ? static_cast<size_t>(D) : static_cast<size_t>(HD);
        float acc[V];
#pragma unroll
        for (int i = 0; i < V; ++i) acc[i] = 0.f;
        float ws = 0.f;
        bool done = false;
        if constexpr (V * sizeof(T) >= 4) {
            if (p.buf) {
                const uint32_t lane_off =
                    static_cast<uint32_t>(base - value) * static_cast<uint32_t>(sizeof(T));  // < val_bytes < 2^31
                gather_sum_buf<T, V, NB>(cw + r * S, S, sg, SG, buffer_of(value, p.val_bytes), lane_off, acc, ws);
                done = true;
            }
        }
        if (!done) gather_sum<T, V, NB>(cw + r * S, S, sg, SG, base, stride, acc, ws);
        for (int m = DV; m < GS; m <<= 1) {
#pragma unroll
            for (int i = 0; i < V; ++i) acc[i] += xor_lane(acc[i], m);
        }
        if (sg == 0 && valid) IO::store(out + static_cast<size_t>(row) * D + ch * V, acc);
    }
}

// float64: float64 accumulation, scalar loads.
template <int WAVES>
__global__ __launch_bounds__(WAVES* kWave) void sample_f64_kernel(SampleParams p) {
    constexpr int NTH = WAVES * kWave;
    const Geom& g = p.g;
    const int LP = g.LP, S = 4 * LP, D = g.D, HD = g.H * D, RB = p.RB;
    extern __shared__ __align__(16) unsigned char smem[];
    Corner<double>* cw = reinterpret_cast<Corner<double>*>(smem);
    const double* __restrict__ value = static_cast<const double*>(p.value);
    const double* __restrict__ loc = static_cast<const double*>(p.loc);
    const double* __restrict__ attn = static_cast<const double*>(p.attn);
    double* __restrict__ out = static_cast<double*>(p.out);
    const int tid = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * RB;
    for (int i = tid; i < RB * LP; i += NTH) {
        const int r = i / LP, j = i - r * LP;
        const int64_t row = row0 + r;
        Corner<double>* c4 = cw + r * S + 4 * j;
        if (row < p.rows) {
            corner4<double, double, true>(loc, attn, g, row, j, c4);
        } else {
            for (int k = 0; k < 4; ++k) c4[k] = Corner<double>{-1, 0.0};
        }
    }
    __syncthreads();
    const int64_t QH = static_cast<int64_t>(g.Q) * g.H;
    for (int it = tid; it < RB * D; it += NTH) {
        const int r = it / D, d = it - r * D;
        const int64_t row = row0 + r;
        if (row >= p.rows) continue;
        const int64_t b = row / QH;
        const int h = static_cast<int>(row % g.H);
        const double* base = g.value_hm ? value + (static_cast<size_t>(b) * g.H + h) * g.N * D + d
                                        : value + static_cast<size_t>(b) * g.N * HD + static_cast<size_t>(h) * D + d;
        const size_t stride = g.value_hm ? static_cast<size_t>(D) : static_cast<size_t>(HD);
        double acc = 0.0;
        for (int s = 0; s < S; ++s) {
            const Corner<double> c = cw[r * S + s];
            const double v = base[static_cast<size_t>(c.tok < 0 ? 0 : c.tok) * stride];
            acc = fma(c.w, c.tok < 0 ? 0.0 : v, acc);
        }
        out[static_cast<size_t>(row) * D + d] = acc;
    }
}

constexpr size_t kLdsBudget = 65536;

inline bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

template <typename T, int V, int WAVES, int NB>
int go_nb(const SampleParams& p, size_t lds, hipStream_t stream) {
    if (p.g.general())
        hipLaunchKernelGGL((sample_kernel<T, V, WAVES, NB, true>), dim3(static_cast<unsigned>(p.per_xcd) * kXcds),
                           dim3(WAVES * kWave), lds, stream, p);
    else
        hipLaunchKernelGGL((sample_kernel<T, V, WAVES, NB, false>), dim3(static_cast<unsigned>(p.per_xcd) * kXcds),
                           dim3(WAVES * kWave), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "sample launch failed: %s", hipGetErrorString(e));
}

template <typename T, int V, int WAVES>
int go(SampleParams p, size_t lds, hipStream_t stream) {
    const int64_t blocks = (p.rows + p.RB - 1) / p.RB;
    p.blocks = static_cast<int>(blocks);
    p.per_xcd = static_cast<int>((blocks + kXcds - 1) / kXcds);
    // corner loads in flight per lane: 8, or 6 when a lane's corners (4 L P / SG) are a multiple of 6 but not of 8,
    // so that no batch carries empty slots
    // (RT-DETR's 12 samples over 4 corner groups: bf16 B8 Q300 7.87 -> 7.01 µs, fp16 B1 Q300 3.69 -> 3.51)
    const int per = 4 * p.g.LP / p.SG;
    const int nb = per % 8 != 0 && per % 6 == 0 ? 6 : 8;
    return nb == 6 ? go_nb<T, V, WAVES, 6>(p, lds, stream) : go_nb<T, V, WAVES, 8>(p, lds, stream);
}

template <typename T, int V>
int go_waves(SampleParams p, int waves, size_t lds, hipStream_t stream) {
    switch (waves) {
        case 1: return go<T, V, 1>(p, lds, stream);
        case 2: return go<T, V, 2>(p, lds, stream);
        case 4: return go<T, V, 4>(p, lds, stream);
        default: return set_error(-1, "sample: waves must be 1, 2 or 4 (got %d)", waves);
    }
}

template <typename T>
int launch_sample_t(SampleParams p, hipStream_t stream, const SampleTune& tune) {
    const Geom& g = p.g;
    const int LP = g.LP, S = 4 * LP, D = g.D;
    constexpr int VMAX = 16 / static_cast<int>(sizeof(T));
    const uintptr_t align = reinterpret_cast<uintptr_t>(p.value) | reinterpret_cast<uintptr_t>(p.out);
    int V = tune.vec > 0 ? tune.vec : VMAX;
    while (V > 1 && (D % V != 0 || align % (V * sizeof(T)) != 0)) V >>= 1;
    if (V > VMAX || D % V != 0 || align % (V * sizeof(T)) != 0)
        return set_error(-1, "sample: %d elements per load do not fit D=%d and the pointer alignment", V, D);
    const int DV = D / V;
    // Launch shape (measured on MI355X): small problems want 8 corner groups per row and 2-wave workgroups, large
    // ones (>= 12k rows) 4 corner groups and 1-wave workgroups; at least 4 corners per lane. Self-attention shapes
    // (queries as many as half the tokens: encoder layers, whose queries are the tokens in order and sample around
    // themselves) want 2 corner groups and 4-wave workgroups, 32 rows of neighbouring queries sharing a CU's L1
    // (DINO encoder B2: 96.9 against 105.5 µs; a B16 decoder of 115k rows keeps the large shape: 48.6 against 50.1).
    const bool big = p.rows >= 12000;
    const bool self_attn = 2 * static_cast<int64_t>(g.Q) >= g.N && big;
    int sg = tune.sg;
    if (sg <= 0) {
        sg = 1;
        if (is_pow2(DV) && DV < kWave) {
            const int cap = self_attn ? 2 : big ? 4 : 8;
            sg = kWave / DV < cap ? kWave / DV : cap;
            while (sg > 1 && S / sg < 4) sg >>= 1;
        }
    }
    if (sg > 1 && !(is_pow2(DV) && is_pow2(sg) && DV * sg <= kWave)) sg = 1;
    const int GS = DV * sg;
    int waves = tune.waves;
    if (waves <= 0) waves = self_attn ? 4 : big ? 1 : 2;
    const int nth = waves * kWave;
    int rb = nth / GS;
    if (rb < 1) rb = 1;
    auto lds = [&](int r) { return static_cast<size_t>(r) * S * sizeof(Corner<float>); };
    while (rb > 1 && lds(rb) > kLdsBudget) --rb;
    p.RB = rb;
    p.SG = sg;
    // Multiply-high divisions instead of the division routines (sampler alone, graph-timed µs, same outputs):
    // bf16 B8 Q300 8.84 -> 7.87, DINO fp16 B4 Q900 12.79 -> 11.09, C = 1024 B2 Q300 23.64 -> 20.84, DINO encoder
    // B2 86.9 -> 76.1; the kernel issues more VALU instructions than anything else bounds it.
    if (LP > 0) p.d_lp = make_fastdiv(static_cast<uint32_t>(LP));
    if (g.P > 0) p.d_p = make_fastdiv(static_cast<uint32_t>(g.P));
    p.d_gs = make_fastdiv(static_cast<uint32_t>(GS));
    p.d_dv = make_fastdiv(static_cast<uint32_t>(DV));
    p.fast = p.rows < (int64_t{1} << 31) && g.H > 0 && g.Q > 0 ? 1 : 0;
    const int64_t val_bytes = static_cast<int64_t>(g.B) * g.N * g.H * D * static_cast<int64_t>(sizeof(T));
    p.buf = V * static_cast<int>(sizeof(T)) >= 4 && val_bytes > 0 && val_bytes < (int64_t{1} << 31) ? 1 : 0;
    p.val_bytes = p.buf ? static_cast<int>(val_bytes) : 0;
    if (p.fast) {
        p.d_h = make_fastdiv(static_cast<uint32_t>(g.H));
        p.d_q = make_fastdiv(static_cast<uint32_t>(g.Q));
        p.d_qh = make_fastdiv(static_cast<uint32_t>(g.Q * g.H));
    }
    // Rows in (b, h, q) order when one image's values exceed an XCD's 4 MB L2 well and each head's rows are read
    // again and again: taking the rows of all heads of a few queries, an XCD's workgroups touch the whole image's
    // values (N * H * D elements), while head by head they touch one head's (N * D) at a time, which then stays in
    // L2 for the Q * L * P * 4 corner reads of that head. Measured on MI355X (sampler alone, graph-timed µs,
    // (b, q, h) -> (b, h, q)), with image = N * H * D * s and reads per row = 4 Q L P / N:
    //  * C = 1024 (44.6 MB; 3.5 and 10.6 reads per row): B2 Q300 30.7 -> 23.7, Q900 75.6 -> 56.7, B1 Q300 17.3 -> 13.4;
    //    at Q50 (0.6 reads per row) 7.77 -> 7.84;
    //  * DINO 4-level (11.4 MB in 16 bits, 22.8 MB in float32): at Q900 (2.6 reads per row) fp16 B2 7.90 -> 7.70, B4
    //    13.5 -> 12.6, B8 23.6 -> 23.0, B16 42.4 -> 40.2, bf16 B4 13.9 -> 13.8, fp32 B4 20.7 -> 19.8; at Q300 (0.9)
    //    fp16 B1 4.2 -> 4.7, B4 6.6 -> 6.9, B8 9.6 -> 10.5;
    //  * 8.6 MB (C = 512 in 16 bits, RT-DETR float32): slower at 1.7 and 5.1 reads per row (C = 512 B4 Q900 20.3 ->
    //    22.9, fp32 B8 Q300 12.7 -> 14.2); 4.3 MB (RT-DETR 16-bit) slower (bf16 B8 9.0 -> 9.6); self-attention
    //    slower (DINO encoder 85 -> 91).
    const int64_t image_bytes = static_cast<int64_t>(g.N) * g.H * D * static_cast<int64_t>(sizeof(T));
    p.hq = !self_attn && image_bytes >= (int64_t{10} << 20) && 2 * static_cast<int64_t>(g.Q) * LP >= g.N ? 1 : 0;
    if (tune.plan != nullptr) {
        const int per = 4 * LP / sg;
        *tune.plan = LaunchPlan{{(p.rows + rb - 1) / rb, waves, rb, sg, V, p.hq, per % 8 != 0 && per % 6 == 0 ? 6 : 8}};
        return 0;
    }
    switch (V) {
        case 1: return go_waves<T, 1>(p, waves, lds(rb), stream);
        case 2: return go_waves<T, 2>(p, waves, lds(rb), stream);
        case 4: return go_waves<T, 4>(p, waves, lds(rb), stream);
        case 8:
            if constexpr (VMAX >= 8) return go_waves<T, 8>(p, waves, lds(rb), stream);
            break;
        default: break;
    }
    return set_error(-1, "sample: unsupported vector width %d", V);
}

int launch_sample_f64(SampleParams p, hipStream_t stream, LaunchPlan* plan) {
    const int S = 4 * p.g.LP;
    int rb = 4;
    while (rb > 1 && static_cast<size_t>(rb) * S * sizeof(Corner<double>) > kLdsBudget) --rb;
    p.RB = rb;
    p.SG = 1;
    const int64_t blocks = (p.rows + rb - 1) / rb;
    if (plan != nullptr) {
        *plan = LaunchPlan{{blocks, 4, rb, 1, 1, 0, 1}};
        return 0;
    }
    hipLaunchKernelGGL((sample_f64_kernel<4>), dim3(static_cast<unsigned>(blocks)), dim3(4 * kWave),
                       static_cast<size_t>(rb) * S * sizeof(Corner<double>), stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "sample launch failed: %s", hipGetErrorString(e));
}

}  // namespace

int launch_sample(int dtype, const void* value, const Geom& g, const void* loc, const void* attn, void* out,
                  hipStream_t stream, const SampleTune& tune) {
    SampleParams p{value, loc, attn, out, g, 1, 1, static_cast<int64_t>(g.B) * g.Q * g.H, 0, 0};
    switch (dtype) {
        case kF32: return launch_sample_t<float>(p, stream, tune);
        case kF16: return launch_sample_t<f16>(p, stream, tune);
        case kBF16: return launch_sample_t<bf16>(p, stream, tune);
        case kF64: return launch_sample_f64(p, stream, tune.plan);
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
}

}  // namespace td
