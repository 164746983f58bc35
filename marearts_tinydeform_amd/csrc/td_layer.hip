// Standalone query prologue of the decoder layer (the computation is described in td_prologue.h): one workgroup per
// (b, tile of QT queries, h) computes the tile's sampling offsets and attention logits for head h (on MFMA for
// 16/32-bit types with 16-byte rows, on the vector ALUs otherwise), the softmax and the reference-point arithmetic,
// and writes locations [B, Q, H, L, P, 2] and attention weights [B, Q, H, L, P] in the accumulation type.
//
// Project mode of the layer runs it before the sampling kernel; fused mode runs it only when the layer kernel
// (the prologue inside the fused kernel) cannot take the problem (float64, unaligned rows).
#include "td_internal.h"

namespace td {
namespace {

struct PrologueParams {
    LayerArgs lay;
    Geom g;
    int QT, qtiles;
    int per_xcd, units;  // workgroup i takes unit (i % 8) * per_xcd + i / 8: a contiguous range per XCD
};

template <typename T, int WAVES, bool MFMA>
__global__ __launch_bounds__(WAVES* kWave) void layer_prologue_kernel(PrologueParams p) {
    using A = typename AccOf<T>::type;
    constexpr int NTH = WAVES * kWave;
    const Geom& g = p.g;
    const int LP = g.LP, QT = p.QT;
    const int XP = p.lay.Cq + 4;
    const int PP = ((3 * LP + 15) & ~15) + 4;
    extern __shared__ __align__(16) unsigned char smem[];
    A* xs = reinterpret_cast<A*>(smem);  // [QT][XP] query rows (+ position embeddings)
    A* pro = xs + QT * XP;               // [16][PP] projections
    A* rstat = pro + 16 * PP;            // [16][2] softmax max, 1 / sum

    const int unit = static_cast<int>(blockIdx.x % kXcds) * p.per_xcd + static_cast<int>(blockIdx.x / kXcds);
    if (unit >= p.units) return;
    const int h = unit % g.H, rest = unit / g.H;
    const int qt = rest % p.qtiles, b = rest / p.qtiles;
    const int q0 = qt * QT;

    stage_queries<T, A, MFMA, NTH>(p.lay, b, q0, QT, g.Q, xs, XP);
    __syncthreads();
    if constexpr (MFMA)
        prologue_mfma<T, WAVES>(p.lay, h, LP, QT, xs, XP, pro, PP);
    else
        prologue_valu<T, A, WAVES>(p.lay, h, LP, QT, xs, XP, pro, PP);
    __syncthreads();
    prologue_stats<A, NTH>(LP, QT, pro, PP, rstat);
    __syncthreads();
    for (int i = static_cast<int>(threadIdx.x); i < QT * LP; i += NTH) {
        const int r = i / LP, j = i - r * LP, q = q0 + r;
        if (q >= g.Q) continue;
        A lx, ly, w;
        prologue_sample<T, A>(p.lay, g, b, q, h, r, j, pro, PP, rstat, lx, ly, w);
    }
}

// Second half of the GEMM route (launch_prologue_gemm): loc_out holds the raw offsets [rows, LP, 2] and attn_out
// the raw logits [rows, LP] (rows = (b, q, h)); each wavefront turns 64 / SEG rows in place into locations and
// softmax weights (SEG = the power of two >= LP lanes per row, lane j of a segment taking sample j).
template <typename T>
__global__ __launch_bounds__(256) void layer_finalize_kernel(LayerArgs a, Geom g, int seg_log2) {
    const int SEG = 1 << seg_log2, lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int64_t row = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * (kWave >> seg_log2) +
                        (lane >> seg_log2);
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
    const int j = lane & (SEG - 1), LP = g.LP;
    const bool on = row < rows && j < LP;
    float* lg = static_cast<float*>(a.attn_out) + row * LP;
    float* off = static_cast<float*>(a.loc_out) + row * LP * 2;
    float x = -INFINITY, ox = 0.f, oy = 0.f;
    if (on) {
        x = lg[j];
        ox = off[2 * j];
        oy = off[2 * j + 1];
    }
    float m = x;
    for (int k = SEG >> 1; k > 0; k >>= 1) m = fmaxf(m, xor_lane(m, k));
    const float e = on ? exp_acc(x - m) : 0.f;
    float sum = e;
    for (int k = SEG >> 1; k > 0; k >>= 1) sum += xor_lane(sum, k);
    if (!on) return;
    lg[j] = e * (1.f / sum);
    const int q = static_cast<int>((row / g.H) % g.Q), b = static_cast<int>(row / (static_cast<int64_t>(g.H) * g.Q));
    float lx, ly;
    layer_location<T, float>(a, g, b, q, j / g.P, ox, oy, lx, ly);
    off[2 * j] = lx;
    off[2 * j + 1] = ly;
}

// The in-place finalize of the GEMM route's raw offsets and logits (layer_finalize_kernel).
template <typename T>
int finalize_prologue(const LayerArgs& la, const Geom& g, hipStream_t stream) {
    int seg_log2 = 0;
    while ((1 << seg_log2) < g.LP) ++seg_log2;
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H, per_wave = kWave >> seg_log2,
                  waves = (rows + per_wave - 1) / per_wave;
    hipLaunchKernelGGL(layer_finalize_kernel<T>, dim3(static_cast<unsigned>((waves + 3) / 4)), dim3(256), 0, stream,
                       la, g, seg_log2);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "layer prologue launch failed: %s", hipGetErrorString(e));
}

// The prologue as two projections on the GEMM (x . W^T computed as hidden . W^T + pos . W^T, float32 out, straight
// into loc_out and attn_out) and the in-place finalize. A workgroup of the single-kernel prologue owns 16 queries of
// one head and streams that head's weights once per 16 queries, so for large problems the weights are read
// B * Q / 16 times; the GEMM tiles 64 queries x 64 outputs and keeps them in LDS. Returns 1, launching nothing,
// when the GEMM cannot take the operands.
template <typename T>
int launch_prologue_gemm(const LayerArgs& la, const Geom& g, hipStream_t stream) {
    constexpr int V = 16 / static_cast<int>(sizeof(T));
    const uintptr_t al = reinterpret_cast<uintptr_t>(la.query) | reinterpret_cast<uintptr_t>(la.pos) |
                         reinterpret_cast<uintptr_t>(la.off_w) | reinterpret_cast<uintptr_t>(la.aw_w) |
                         reinterpret_cast<uintptr_t>(la.loc_out) | reinterpret_cast<uintptr_t>(la.attn_out);
    if (la.Cq <= 0 || la.Cq % V != 0 || al % 16 != 0 || g.P <= 0) return 1;
    const int64_t M = static_cast<int64_t>(g.B) * g.Q, NO = static_cast<int64_t>(g.H) * g.LP;
    const int dt = std::is_same<T, float>::value ? kF32 : std::is_same<T, f16>::value ? kF16 : kBF16;
    int rc = launch_proj_f32_pair(dt, la.query, la.pos, la.off_w, la.off_b, static_cast<float*>(la.loc_out), 2 * NO,
                                  la.aw_w, la.aw_b, static_cast<float*>(la.attn_out), NO, M, la.Cq, stream, &la, &g);
    if (rc < 0) return rc;
    if (rc == 2) return 0;  // finalized in the projections' epilogue
    if (rc == 0) return finalize_prologue<T>(la, g, stream);
    rc = launch_proj_f32(dt, la.query, la.pos, la.off_w, la.off_b, static_cast<float*>(la.loc_out), M, la.Cq, 2 * NO,
                         stream);
    if (rc != 0) return rc;
    rc = launch_proj_f32(dt, la.query, la.pos, la.aw_w, la.aw_b, static_cast<float*>(la.attn_out), M, la.Cq, NO,
                         stream);
    if (rc != 0) return rc;
    return finalize_prologue<T>(la, g, stream);
}

constexpr size_t kLdsBudget = 65536;

template <typename T, bool MFMA>
int go(PrologueParams p, size_t lds, hipStream_t stream) {
    const int64_t units = static_cast<int64_t>(p.g.B) * p.qtiles * p.g.H;
    p.units = static_cast<int>(units);
    p.per_xcd = static_cast<int>((units + kXcds - 1) / kXcds);
    hipLaunchKernelGGL((layer_prologue_kernel<T, 4, MFMA>), dim3(static_cast<unsigned>(p.per_xcd) * kXcds),
                       dim3(4 * kWave), lds, stream, p);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "layer prologue launch failed: %s", hipGetErrorString(e));
}

template <typename T>
int launch_prologue_t(PrologueParams p, hipStream_t stream) {
    using A = typename AccOf<T>::type;
    const LayerArgs& la = p.lay;
    const int Cq = la.Cq, LP = p.g.LP, PP = ((3 * LP + 15) & ~15) + 4;
    bool mfma = false;
    if constexpr (!std::is_same<T, double>::value) {
        constexpr int V = 16 / static_cast<int>(sizeof(T));
        auto al = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
        mfma = Cq > 0 && Cq % V == 0 && al(la.query) && al(la.off_w) && al(la.aw_w) && (la.pos == nullptr || al(la.pos));
    }
    auto lds = [&](int q) { return (static_cast<size_t>(q) * (Cq + 4) + 16 * PP + 32) * sizeof(A); };
    int qt = p.g.Q < 16 ? p.g.Q : 16;
    if (qt < 1) qt = 1;
    while (qt > 1 && lds(qt) > kLdsBudget) --qt;
    if (lds(qt) > kLdsBudget)
        return set_error(-1, "layer prologue: %d query channels do not fit the LDS budget", Cq);
    p.QT = qt;
    p.qtiles = (p.g.Q + qt - 1) / qt;
    if constexpr (!std::is_same<T, double>::value) {
        if (mfma) return go<T, true>(p, lds(qt), stream);
    }
    return go<T, false>(p, lds(qt), stream);
}

}  // namespace

bool prologue_wants_gemm(int dtype, const Geom& g, int64_t Cq) {
    const double macs = static_cast<double>(g.B) * g.Q * g.H * 3 * g.LP * Cq;
    return dtype != kF64 && macs >= 8e8;
}

int launch_prologue(int dtype, const LayerArgs& layer, const Geom& g, hipStream_t stream, int route) {
    if (layer.loc_out == nullptr || layer.attn_out == nullptr)
        return set_error(-1, "layer prologue: locations and weights need output buffers");
    // route 0: by the projections' multiply-adds. Measured on MI355X: the single kernel up to DINO-sized problems
    // (3600 queries, Cq 256, 8 heads x 16 samples, 3.5e8: 14-17 µs against 25 µs for the GEMM route), the GEMM route
    // for the C = 1024 shape (600 queries, 16 heads x 64 samples, 1.9e9: 45 µs against 72 µs).
    if (dtype != kF64 && (route == 2 || (route == 0 && prologue_wants_gemm(dtype, g, layer.Cq)))) {
        int rc = 1;
        switch (dtype) {
            case kF32: rc = launch_prologue_gemm<float>(layer, g, stream); break;
            case kF16: rc = launch_prologue_gemm<f16>(layer, g, stream); break;
            case kBF16: rc = launch_prologue_gemm<bf16>(layer, g, stream); break;
            default: break;
        }
        if (rc <= 0) return rc;  // launched, or failed; 1: the GEMM cannot take the operands
    }
    PrologueParams p{layer, g, 1, 1, 0, 0};
    switch (dtype) {
        case kF32: return launch_prologue_t<float>(p, stream);
        case kF16: return launch_prologue_t<f16>(p, stream);
        case kBF16: return launch_prologue_t<bf16>(p, stream);
        case kF64: return launch_prologue_t<double>(p, stream);
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
}

}  // namespace td
