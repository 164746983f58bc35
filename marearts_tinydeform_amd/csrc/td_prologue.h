// Query prologue of a deformable-attention decoder layer, shared by the fused layer kernel (where it feeds the
// corner table directly) and the standalone prologue kernel (which writes locations and weights out).
//
// Restates HF transformers RTDetrMultiscaleDeformableAttention.forward (models/rt_detr/modeling_rt_detr.py:673-713)
// for the query rows q of image b and one head h, with LP = L * P samples per head:
//   x        = hidden[b, q] (+ position_embeddings[b, q])
//   off[n]   = Woff[h*2LP + n] . x + boff[h*2LP + n]       n < 2 LP   (sample n / 2, coordinate n % 2)
//   logit[j] = Wattn[h*LP + j] . x + battn[h*LP + j]       j < LP
//   a[j]     = softmax over j of logit
//   loc[j]   = ref[b, q, l'] + off[j] / (W_l, H_l)                          reference points of 2 coordinates
//            = ref[b, q, l', 0:2] + off[j] / P * ref[b, q, l', 2:4] * 0.5   4 coordinates (box centre, size)
// with l = j / P the sample's level and l' = l when the reference points carry L levels, 0 when they carry one.
// Everything is computed in float32 (float64 for float64 tensors) and never rounded to the element type, so the
// locations keep full precision into the corner rule.
#pragma once

#include "td_common.h"

namespace td {

struct LayerArgs {
    const void* query = nullptr;  // [B, Q, Cq] hidden states of the queries
    const void* pos = nullptr;    // [B, Q, Cq] position embeddings, or null
    const void* ref = nullptr;    // [B, Q, RL, RD] reference points
    const void* off_w = nullptr;  // [H * LP * 2, Cq] sampling-offset projection
    const void* off_b = nullptr;  // [H * LP * 2] or null
    const void* aw_w = nullptr;   // [H * LP, Cq] attention-weight projection
    const void* aw_b = nullptr;   // [H * LP] or null
    void* loc_out = nullptr;      // [B, Q, H, LP, 2] in the accumulation type, or null
    void* attn_out = nullptr;     // [B, Q, H, LP] in the accumulation type, or null
    int Cq = 0, RL = 1, RD = 2;
};

__device__ __forceinline__ float exp_acc(float x) { return expf(x); }
__device__ __forceinline__ double exp_acc(double x) { return exp(x); }

template <typename T>
struct MfmaOp;
template <>
struct MfmaOp<f16> {
    typedef f16x8 frag;
    __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};
template <>
struct MfmaOp<bf16> {
    typedef bf16x8 frag;
    __device__ __forceinline__ static f32x4 mma(frag a, frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};

// x rows of the tile (queries q0 .. q0 + QT - 1 of image b) into LDS in the accumulation type, row pitch XP.
// VEC: 16-byte loads (Cq a multiple of 16 bytes, 16-byte aligned query and position rows).
template <typename T, typename A, bool VEC, int NTH>
__device__ __forceinline__ void stage_queries(const LayerArgs& a, int b, int q0, int QT, int Q, A* xs, int XP) {
    const T* __restrict__ hq = static_cast<const T*>(a.query);
    const T* __restrict__ hp = static_cast<const T*>(a.pos);
    const int Cq = a.Cq;
    if constexpr (VEC) {
        constexpr int V = 16 / static_cast<int>(sizeof(T));
        using IO = VecIO<T, V>;
        const int CV = Cq / V;
        for (int i = threadIdx.x; i < QT * CV; i += NTH) {
            const int r = i / CV, c = (i - r * CV) * V, q = q0 + r;
            float v[V];
#pragma unroll
            for (int e = 0; e < V; ++e) v[e] = 0.f;
            if (q < Q) {
                const size_t o = (static_cast<size_t>(b) * Q + q) * Cq + c;
                IO::unpack(IO::load(hq + o), v);
                if (hp != nullptr) {
                    float u[V];
                    IO::unpack(IO::load(hp + o), u);
#pragma unroll
                    for (int e = 0; e < V; ++e) v[e] += u[e];
                }
            }
#pragma unroll
            for (int e = 0; e < V; ++e) xs[r * XP + c + e] = v[e];
        }
    } else {
        for (int i = threadIdx.x; i < QT * Cq; i += NTH) {
            const int r = i / Cq, c = i - r * Cq, q = q0 + r;
            A v = 0;
            if (q < Q) {
                const size_t o = (static_cast<size_t>(b) * Q + q) * Cq + c;
                v = cvt<A>(hq[o]);
                if (hp != nullptr) v += cvt<A>(hp[o]);
            }
            xs[r * XP + c] = v;
        }
    }
}

// Weight row and bias of projection column n of head h (n < 2 LP: sampling offsets; then attention logits).
template <typename T>
__device__ __forceinline__ const T* proj_row(const LayerArgs& a, int h, int LP, int n) {
    return n < 2 * LP ? static_cast<const T*>(a.off_w) + (static_cast<size_t>(h) * 2 * LP + n) * a.Cq
                      : static_cast<const T*>(a.aw_w) + (static_cast<size_t>(h) * LP + n - 2 * LP) * a.Cq;
}
template <typename T, typename A>
__device__ __forceinline__ A proj_bias(const LayerArgs& a, int h, int LP, int n) {
    const T* ob = static_cast<const T*>(a.off_b);
    const T* ab = static_cast<const T*>(a.aw_b);
    if (n < 2 * LP) return ob != nullptr ? cvt<A>(ob[static_cast<size_t>(h) * 2 * LP + n]) : static_cast<A>(0);
    return ab != nullptr ? cvt<A>(ab[static_cast<size_t>(h) * LP + n - 2 * LP]) : static_cast<A>(0);
}

// pro[r * PP + n] = projection column n of x row r (bias included) for r < 16, n < 3 LP, on MFMA: one 16 x 16
// output tile per job, jobs spread over the wavefronts. Rows r >= QT multiply zeros. 16-bit types split x into
// hi + lo halves (two MFMAs per K block) so the float32 sum x = hidden + pos loses nothing to the input rounding.
// Needs Cq a multiple of 16 bytes and 16-byte aligned weights; XP a multiple of 4.
template <typename T, int WAVES>
__device__ __forceinline__ void prologue_mfma(const LayerArgs& a, int h, int LP, int QT, const float* xs, int XP,
                                              float* pro, int PP) {
    const int Cq = a.Cq, NP = 3 * LP, NT0 = (NP + 15) >> 4;
    const int wave = static_cast<int>(threadIdx.x) / kWave, lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int n16 = lane & 15, kg = lane >> 4;
    const bool av = n16 < QT;
    const float* xa = xs + (av ? n16 : 0) * XP;
    for (int nt = wave; nt < NT0; nt += WAVES) {
        const int n = nt * 16 + n16;
        const bool nv = n < NP;
        const T* wr = proj_row<T>(a, h, LP, nv ? n : 0);
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        // the weight row streams from L2/HBM: KB K blocks of loads are issued before the first is used, so a
        // wavefront waits one memory latency per KB blocks rather than per block
        constexpr int KB = 8;
        if constexpr (sizeof(T) == 2) {
            using M = MfmaOp<T>;
            using frag = typename M::frag;
            for (int k0 = 0; k0 < Cq; k0 += 32 * KB) {
                u32x4 braw[KB];
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    const int k = k0 + u * 32 + kg * 8;
                    braw[u] = (nv && k < Cq) ? *reinterpret_cast<const u32x4*>(wr + k) : u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    const int k = k0 + u * 32 + kg * 8;
                    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0;
                    if (av && k < Cq) {
                        a0 = *reinterpret_cast<const f32x4*>(xa + k);
                        a1 = *reinterpret_cast<const f32x4*>(xa + k + 4);
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
                    const frag bf = __builtin_bit_cast(frag, braw[u]);
                    acc = M::mma(hi, bf, acc);
                    acc = M::mma(lo, bf, acc);
                }
            }
        } else {
            for (int k0 = 0; k0 < Cq; k0 += 16 * KB) {
                f32x4 bq[KB];
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    const int k = k0 + u * 16 + kg * 4;
                    bq[u] = (nv && k < Cq) ? *reinterpret_cast<const f32x4*>(wr + k) : f32x4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int u = 0; u < KB; ++u) {
                    const int k = k0 + u * 16 + kg * 4;
                    f32x4 aq = {0.f, 0.f, 0.f, 0.f};
                    if (av && k < Cq) aq = *reinterpret_cast<const f32x4*>(xa + k);
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(aq[j], bq[u][j], acc, 0, 0, 0);
                }
            }
        }
        const float bn = nv ? proj_bias<T, float>(a, h, LP, n) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) pro[(4 * kg + i) * PP + nt * 16 + n16] = acc[i] + bn;
    }
}

// The same projection on the vector ALUs for any Cq and alignment (and float64): one wavefront-wide dot product
// per (row, column), rows r < QT only.
template <typename T, typename A, int WAVES>
__device__ __forceinline__ void prologue_valu(const LayerArgs& a, int h, int LP, int QT, const A* xs, int XP, A* pro,
                                              int PP) {
    const int Cq = a.Cq, NP = 3 * LP;
    const int wave = static_cast<int>(threadIdx.x) / kWave, lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    for (int o = wave; o < QT * NP; o += WAVES) {  // uniform across the wavefront
        const int r = o / NP, n = o - r * NP;
        const T* wr = proj_row<T>(a, h, LP, n);
        A s = 0;
        for (int c = lane; c < Cq; c += kWave) s = fma(cvt<A>(wr[c]), xs[r * XP + c], s);
        s = wave_sum(s);
        if (lane == 0) pro[r * PP + n] = s + proj_bias<T, A>(a, h, LP, n);
    }
}

// Softmax statistics of the attention logits of rows r < QT: rstat[2r] = max, rstat[2r + 1] = 1 / sum of exp.
template <typename A, int NTH>
__device__ __forceinline__ void prologue_stats(int LP, int QT, const A* pro, int PP, A* rstat) {
    for (int r = static_cast<int>(threadIdx.x); r < QT; r += NTH) {
        const A* lg = pro + r * PP + 2 * LP;
        A m = lg[0];
        for (int j = 1; j < LP; ++j) m = fmax(m, lg[j]);
        A s = 0;
        for (int j = 0; j < LP; ++j) s += exp_acc(lg[j] - m);
        rstat[2 * r] = m;
        rstat[2 * r + 1] = static_cast<A>(1) / s;
    }
}

// Reference-point arithmetic: location (lx, ly) of a sample on level l of query q of image b from its offsets
// (ox, oy).
template <typename T, typename A>
__device__ __forceinline__ void layer_location(const LayerArgs& a, const Geom& g, int b, int q, int l, A ox, A oy,
                                               A& lx, A& ly) {
    const T* rp = static_cast<const T*>(a.ref) +
                  ((static_cast<size_t>(b) * g.Q + q) * a.RL + (a.RL == 1 ? 0 : l)) * a.RD;
    const A rx = cvt<A>(rp[0]), ry = cvt<A>(rp[1]);
    if (a.RD == 2) {
        lx = rx + ox / static_cast<A>(g.shapes[2 * l + 1]);
        ly = ry + oy / static_cast<A>(g.shapes[2 * l]);
    } else {
        lx = rx + ox / static_cast<A>(g.P) * cvt<A>(rp[2]) * static_cast<A>(0.5);
        ly = ry + oy / static_cast<A>(g.P) * cvt<A>(rp[3]) * static_cast<A>(0.5);
    }
}

// Location (lx, ly) and attention weight w of sample j of tile row r (query q of image b, head h); also stored
// to a.loc_out / a.attn_out when those are set.
template <typename T, typename A>
__device__ __forceinline__ void prologue_sample(const LayerArgs& a, const Geom& g, int b, int q, int h, int r, int j,
                                                const A* pro, int PP, const A* rstat, A& lx, A& ly, A& w) {
    const int LP = g.LP, l = j / g.P;
    w = exp_acc(pro[r * PP + 2 * LP + j] - rstat[2 * r]) * rstat[2 * r + 1];
    layer_location<T, A>(a, g, b, q, l, pro[r * PP + 2 * j], pro[r * PP + 2 * j + 1], lx, ly);
    const size_t idx = ((static_cast<size_t>(b) * g.Q + q) * g.H + h) * LP + j;
    if (a.loc_out != nullptr) {
        A* lo = static_cast<A*>(a.loc_out);
        lo[2 * idx] = lx;
        lo[2 * idx + 1] = ly;
    }
    if (a.attn_out != nullptr) static_cast<A*>(a.attn_out)[idx] = w;
}

}  // namespace td
