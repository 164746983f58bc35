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

int launch_prologue(int dtype, const LayerArgs& layer, const Geom& g, hipStream_t stream) {
    if (layer.loc_out == nullptr || layer.attn_out == nullptr)
        return set_error(-1, "layer prologue: locations and weights need output buffers");
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
