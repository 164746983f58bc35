// Backward of value projection + multi-scale deformable attention (training). The reference operator is inference
// only (README.md:61); the gradients here are those of its reference computation (reference.py:13-40: F.linear, then
// bilinear grid_sample with zero padding, align_corners=False, weighted by the attention), in project order, which
// equals fused order up to rounding:
//
//   value       = memory . W^T + b                                   [B, N, H*D]
//   out[r, :]   = sum_s a_s sum_c w_c(fx_s, fy_s) value[t_c, h*D:(h+1)*D]      r = (b, q, h), s = (l, p), c = corner
//
//   G = grad_value[t, h*D + d] = sum over (r, s, c) hitting t of a_s w_c g_r[d]         (g_r = grad_out[r, :])
//   grad_attn[r, s]  = sum_c w_c d_c                 d_c = value[t_c] . g_r (0 for a corner outside the map)
//   grad_loc[r, s]   = a_s (dV/dfx W_l, dV/dfy H_l)  dV/dfx = (1 - fy)(d_1 - d_0) + fy (d_3 - d_2)
//                                                    dV/dfy = (1 - fx)(d_2 - d_0) + fx (d_3 - d_1)
//   grad_memory = G . W,   grad_W = G^T . memory,   grad_b = sum over tokens of G
//
// (x = loc_x W_l - 0.5, so dx/dloc_x = W_l; corner k has dx = k & 1, dy = k >> 1.) A location clamped to the map's
// guard band has all four corners outside, so its gradient is 0, as for grid_sample's zero padding. Discrete
// sampling (D-FINE) is piecewise constant in the location: its location gradient is 0.
#include "td_gemm_mfma.h"

namespace td {
namespace {

// The bilinear taps of a sample: tokens (-1 outside the map, outside [0, N) or on a padded token) and the
// fractional position (fx, fy); the same rule as corners_at (td_common.h), keeping the two factors apart.
template <typename A>
struct Taps {
    int tok[4];
    A fx, fy;
};

// taps_at_b takes the row's image b (for the padding mask); taps_at derives it from the row index (b, q, h).
template <typename A>
__device__ __forceinline__ Taps<A> taps_at_b(A lx, A ly, int l, const Geom& g, int64_t b) {
    Taps<A> t;
    const int hl = static_cast<int>(g.shapes[2 * l]);
    const int wl = static_cast<int>(g.shapes[2 * l + 1]);
    const int64_t st = g.starts[l];
    if (g.discrete) {
        const A fx = fmin(fmax(lx * static_cast<A>(wl) + static_cast<A>(0.5), static_cast<A>(-1)), static_cast<A>(wl));
        const A fy = fmin(fmax(ly * static_cast<A>(hl) + static_cast<A>(0.5), static_cast<A>(-1)), static_cast<A>(hl));
        int xi = static_cast<int>(fx), yi = static_cast<int>(fy);
        xi = xi < 0 ? 0 : xi > wl - 1 ? wl - 1 : xi;
        yi = yi < 0 ? 0 : yi > hl - 1 ? hl - 1 : yi;
        const int64_t tk = st + static_cast<int64_t>(yi) * wl + xi;
        bool in = wl > 0 && hl > 0 && tk >= 0 && tk < g.N;
        if (in && g.mask != nullptr) in = g.mask[b * g.N + tk] == 0;
        t.tok[0] = in ? static_cast<int>(tk) : -1;
        t.tok[1] = t.tok[2] = t.tok[3] = -1;
        t.fx = t.fy = 0;  // weight 1 on tap 0 (see tap_weight)
        return t;
    }
    A x = lx * static_cast<A>(wl) - static_cast<A>(0.5);
    A y = ly * static_cast<A>(hl) - static_cast<A>(0.5);
    x = fmin(fmax(x, static_cast<A>(-2)), static_cast<A>(wl) + static_cast<A>(1));
    y = fmin(fmax(y, static_cast<A>(-2)), static_cast<A>(hl) + static_cast<A>(1));
    const A xf = floor(x), yf = floor(y);
    const int x0 = static_cast<int>(xf), y0 = static_cast<int>(yf);
    t.fx = x - xf;
    t.fy = y - yf;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int xi = x0 + (k & 1), yi = y0 + (k >> 1);
        const int64_t tk = st + static_cast<int64_t>(yi) * wl + xi;
        bool in = xi >= 0 && xi < wl && yi >= 0 && yi < hl && tk >= 0 && tk < g.N;
        if (in && g.mask != nullptr) in = g.mask[b * g.N + tk] == 0;
        t.tok[k] = in ? static_cast<int>(tk) : -1;
    }
    return t;
}

template <typename A>
__device__ __forceinline__ Taps<A> taps_at(A lx, A ly, int l, const Geom& g, int64_t row) {
    return taps_at_b<A>(lx, ly, l, g, row / (static_cast<int64_t>(g.Q) * g.H));
}

template <typename A>
__device__ __forceinline__ A tap_weight(const Taps<A>& t, int k) {
    return ((k & 1) ? t.fx : static_cast<A>(1) - t.fx) * ((k >> 1) ? t.fy : static_cast<A>(1) - t.fy);
}

__device__ __forceinline__ void atomic_add(float* p, float v) { atomicAdd(p, v); }
__device__ __forceinline__ void atomic_add(double* p, double v) { atomicAdd(p, v); }

template <typename A>
__device__ __forceinline__ A xor_sum(A v, int mask) {
    return v + xor_lane(v, mask);
}

struct BackParams {
    const void* value;
    const void* loc;
    const void* attn;
    const void* grad_out;
    void* grad_value;  // [B, N, H*D] accumulation type, zeroed
    void* grad_loc;    // [rows, LP, 2] element type (accumulation type with g.loc_acc)
    void* grad_attn;   // [rows, LP]
    Geom g;
    int LG;           // lanes per sample: a power of two, LG * CE >= D
    int scatter = 1;  // sample_backward_vec_kernel: 0 leaves the value gradient to scatter_bucket_kernel
};

// One wavefront per row (b, q, h); its LP samples go 64 / LG at a time, LG lanes per sample, lane `sub` of a sample
// owning channels sub, sub + LG, ... (CE of them). The channels are interleaved so that each value-gradient atomic
// instruction adds, for each sample, LG consecutive floats of one token's row (one 128-byte line at D = 32): the L2
// merges them, where a lane-contiguous split would spread one instruction over several lines per sample.
// grad_out's channels are read once per row.
template <typename T, int CE>
__global__ __launch_bounds__(256) void sample_backward_kernel(BackParams p) {
    using A = typename AccOf<T>::type;
    const Geom& g = p.g;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
    if (row >= rows) return;  // uniform across the wavefront
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int LG = p.LG, per = kWave / LG, slot = lane / LG, sub = lane - slot * LG;
    const int D = g.D, HD = g.H * g.D, LP = g.LP;
    const int h = static_cast<int>(row % g.H);
    const int64_t bq = row / g.H, b = bq / g.Q;

    const T* __restrict__ go = static_cast<const T*>(p.grad_out) + bq * HD + h * D;
    A gr[CE];
#pragma unroll
    for (int e = 0; e < CE; ++e) gr[e] = sub + e * LG < D ? cvt<A>(go[sub + e * LG]) : static_cast<A>(0);

    const T* __restrict__ vb = static_cast<const T*>(p.value) + b * g.N * HD + h * D;
    A* __restrict__ gv = static_cast<A*>(p.grad_value) + b * g.N * HD + h * D;
    for (int j0 = 0; j0 < LP; j0 += per) {
        const int j = j0 + slot;
        const bool on = j < LP;  // uniform within a sample's lane group
        A lx = 0, ly = 0, a = 0;
        int l = 0;
        if (on) {
            const int64_t idx = row * LP + j;
            if (g.loc_acc) {
                lx = static_cast<const A*>(p.loc)[2 * idx];
                ly = static_cast<const A*>(p.loc)[2 * idx + 1];
                a = static_cast<const A*>(p.attn)[idx];
            } else {
                lx = cvt<A>(static_cast<const T*>(p.loc)[2 * idx]);
                ly = cvt<A>(static_cast<const T*>(p.loc)[2 * idx + 1]);
                a = cvt<A>(static_cast<const T*>(p.attn)[idx]);
            }
            l = level_of(g, j);
        }
        Taps<A> t;
        if (on) {
            t = taps_at<A>(lx, ly, l, g, row);
        } else {
            t.tok[0] = t.tok[1] = t.tok[2] = t.tok[3] = -1;
            t.fx = t.fy = 0;
        }
        A d[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            d[k] = 0;
            const int tk = t.tok[k];
            if (tk < 0) continue;
            const A w = g.discrete ? (k == 0 ? static_cast<A>(1) : static_cast<A>(0)) : tap_weight(t, k);
            const A aw = a * w;
            const T* vr = vb + static_cast<int64_t>(tk) * HD;
            A* gr_row = gv + static_cast<int64_t>(tk) * HD;
#pragma unroll
            for (int e = 0; e < CE; ++e) {
                const int c = sub + e * LG;
                if (c < D) {
                    d[k] += cvt<A>(vr[c]) * gr[e];
                    atomic_add(gr_row + c, aw * gr[e]);
                }
            }
        }
        // d_k over the sample's LG lanes (xor within the lane group)
        for (int m = LG >> 1; m > 0; m >>= 1) {
#pragma unroll
            for (int k = 0; k < 4; ++k) d[k] = xor_sum(d[k], m);
        }
        if (on && sub == 0) {
            const int64_t idx = row * LP + j;
            A ga, gx = 0, gy = 0;
            if (g.discrete) {
                ga = d[0];
            } else {
                ga = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) ga += tap_weight(t, k) * d[k];
                const A one = 1;
                const A dvx = (one - t.fy) * (d[1] - d[0]) + t.fy * (d[3] - d[2]);
                const A dvy = (one - t.fx) * (d[2] - d[0]) + t.fx * (d[3] - d[1]);
                gx = a * dvx * static_cast<A>(g.shapes[2 * l + 1]);
                gy = a * dvy * static_cast<A>(g.shapes[2 * l]);
            }
            if (g.loc_acc) {
                static_cast<A*>(p.grad_loc)[2 * idx] = gx;
                static_cast<A*>(p.grad_loc)[2 * idx + 1] = gy;
                static_cast<A*>(p.grad_attn)[idx] = ga;
            } else {
                static_cast<T*>(p.grad_loc)[2 * idx] = static_cast<T>(gx);
                static_cast<T*>(p.grad_loc)[2 * idx + 1] = static_cast<T>(gy);
                static_cast<T*>(p.grad_attn)[idx] = static_cast<T>(ga);
            }
        }
    }
}

// The same gradients for D <= 64 (one channel per lane), ordered so that no load waits behind an atomic. A
// wavefront's vector memory operations retire in order, so a load issued after the value-gradient atomics of earlier
// corners cannot be consumed before those atomics have completed at the L2; in sample_backward_kernel each corner's
// value load sits behind the previous corners' atomics. Here the wavefront of row (b, q, h) first computes the taps
// of all its LP samples (lane j: sample j) into LDS, then works through the samples in chunks of NC iterations of
// 64 / LG samples: the chunk's value loads are issued together, and the next chunk's loads are issued before this
// chunk's atomics, so the atomics retire while the next chunk computes.
// location and attention weight of sample idx (= row * LP + j), in the element type or, with g.loc_acc, in the
// accumulation type
template <typename T, typename A>
__device__ __forceinline__ void sample_input(const BackParams& p, int64_t idx, A& lx, A& ly, A& a) {
    if (p.g.loc_acc) {
        lx = static_cast<const A*>(p.loc)[2 * idx];
        ly = static_cast<const A*>(p.loc)[2 * idx + 1];
        a = static_cast<const A*>(p.attn)[idx];
    } else {
        lx = cvt<A>(static_cast<const T*>(p.loc)[2 * idx]);
        ly = cvt<A>(static_cast<const T*>(p.loc)[2 * idx + 1]);
        a = cvt<A>(static_cast<const T*>(p.attn)[idx]);
    }
}

template <typename A>
struct BTap {
    int tok[4];
    A fx, fy, a;
    A wl, hl;  // the sample's level width and height (the location gradient's scale)
};

template <typename T>
__global__ __launch_bounds__(256) void sample_backward_batched_kernel(BackParams p) {
    using A = typename AccOf<T>::type;
    constexpr int NC = 4;  // iterations per chunk
    __shared__ BTap<A> taps[4][kMaxLevelPoints];
    const Geom& g = p.g;
    const int wv = static_cast<int>(threadIdx.x) >> 6;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wv;
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
    if (row >= rows) return;  // uniform across the wavefront; no workgroup barrier below
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int LG = p.LG, per = kWave / LG, slot = lane / LG, sub = lane - slot * LG;
    const int D = g.D, HD = g.H * g.D, LP = g.LP;
    const int h = static_cast<int>(row % g.H);
    const int64_t bq = row / g.H, b = bq / g.Q;
    BTap<A>* tw = taps[wv];

    const T* __restrict__ go = static_cast<const T*>(p.grad_out) + bq * HD + h * D;
    const A gr = sub < D ? cvt<A>(go[sub]) : static_cast<A>(0);

    // taps of every sample of the row, one sample per lane (LP <= 64)
    if (lane < LP) {
        const int64_t idx = row * LP + lane;
        A lx, ly, a;
        sample_input<T, A>(p, idx, lx, ly, a);
        const int l = level_of(g, lane);
        const Taps<A> t = taps_at<A>(lx, ly, l, g, row);
        BTap<A> bt;
#pragma unroll
        for (int k = 0; k < 4; ++k) bt.tok[k] = t.tok[k];
        bt.fx = t.fx;
        bt.fy = t.fy;
        bt.a = a;
        bt.wl = static_cast<A>(g.shapes[2 * l + 1]);
        bt.hl = static_cast<A>(g.shapes[2 * l]);
        tw[lane] = bt;
    }
    // the wavefront's own LDS writes, read back by other lanes of the same wavefront: LDS operations of one
    // wavefront complete in order
    __builtin_amdgcn_wave_barrier();

    const T* __restrict__ vb = static_cast<const T*>(p.value) + b * g.N * HD + h * D + (sub < D ? sub : 0);
    A* __restrict__ gv = static_cast<A*>(p.grad_value) + b * g.N * HD + h * D + sub;
    const int nit = (LP + per - 1) / per;

    // value loads of chunk c0 (iterations c0 .. c0 + NC - 1); corners outside the map read token 0 and are dropped
    auto load = [&](int c0, T (&v)[NC][4]) {
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int j = (c0 + i) * per + slot;
            const bool on = c0 + i < nit && j < LP;
            const BTap<A> t = tw[on ? j : 0];  // unconditional: no branch around the loads
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int tk = on ? t.tok[k] : -1;
                v[i][k] = vb[static_cast<int64_t>(tk < 0 ? 0 : tk) * HD];
            }
        }
    };
    // gradients of chunk c0 from its loaded values: location and weight gradients, then the value-gradient atomics
    auto finish = [&](int c0, const T (&v)[NC][4], auto&& between) {
        A d[NC][4];
        BTap<A> bt[NC];
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int j = (c0 + i) * per + slot;
            const bool on = c0 + i < nit && j < LP;
            bt[i] = tw[on ? j : 0];
            if (!on) bt[i].tok[0] = bt[i].tok[1] = bt[i].tok[2] = bt[i].tok[3] = -1;
#pragma unroll
            for (int k = 0; k < 4; ++k) d[i][k] = bt[i].tok[k] >= 0 ? cvt<A>(v[i][k]) * gr : static_cast<A>(0);
        }
        between();  // the next chunk's loads go out before this chunk's atomics
        for (int m = LG >> 1; m > 0; m >>= 1) {
#pragma unroll
            for (int i = 0; i < NC; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) d[i][k] = xor_sum(d[i][k], m);
        }
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int j = (c0 + i) * per + slot;
            if (!(c0 + i < nit && j < LP) || sub != 0) continue;
            Taps<A> t;
#pragma unroll
            for (int k = 0; k < 4; ++k) t.tok[k] = bt[i].tok[k];
            t.fx = bt[i].fx;
            t.fy = bt[i].fy;
            const A a = bt[i].a;
            const int64_t idx = row * LP + j;
            A ga, gx = 0, gy = 0;
            if (g.discrete) {
                ga = d[i][0];
            } else {
                ga = 0;
#pragma unroll
                for (int k = 0; k < 4; ++k) ga += tap_weight(t, k) * d[i][k];
                const A one = 1;
                const A dvx = (one - t.fy) * (d[i][1] - d[i][0]) + t.fy * (d[i][3] - d[i][2]);
                const A dvy = (one - t.fx) * (d[i][2] - d[i][0]) + t.fx * (d[i][3] - d[i][1]);
                gx = a * dvx * bt[i].wl;
                gy = a * dvy * bt[i].hl;
            }
            if (g.loc_acc) {
                static_cast<A*>(p.grad_loc)[2 * idx] = gx;
                static_cast<A*>(p.grad_loc)[2 * idx + 1] = gy;
                static_cast<A*>(p.grad_attn)[idx] = ga;
            } else {
                static_cast<T*>(p.grad_loc)[2 * idx] = static_cast<T>(gx);
                static_cast<T*>(p.grad_loc)[2 * idx + 1] = static_cast<T>(gy);
                static_cast<T*>(p.grad_attn)[idx] = static_cast<T>(ga);
            }
        }
        if (sub < D) {
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                Taps<A> t;
#pragma unroll
                for (int k = 0; k < 4; ++k) t.tok[k] = bt[i].tok[k];
                t.fx = bt[i].fx;
                t.fy = bt[i].fy;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const int tk = bt[i].tok[k];
                    if (tk < 0) continue;
                    const A w = g.discrete ? (k == 0 ? static_cast<A>(1) : static_cast<A>(0)) : tap_weight(t, k);
                    atomic_add(gv + static_cast<int64_t>(tk) * HD, bt[i].a * w * gr);
                }
            }
        }
    };

    T va[NC][4], vb2[NC][4];
    load(0, va);
    for (int c0 = 0; c0 < nit; c0 += 2 * NC) {
        finish(c0, va, [&] { if (c0 + NC < nit) load(c0 + NC, vb2); });
        if (c0 + NC >= nit) break;
        finish(c0 + NC, vb2, [&] { if (c0 + 2 * NC < nit) load(c0 + 2 * NC, va); });
    }
}

inline bool is_pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int x) { return 31 - __builtin_clz(static_cast<unsigned>(x)); }

// The batched form with 16-byte value loads (16/32-bit types, D * element size a multiple of 16, D <= 64). The
// corner dot products d_c = value[t_c] . g_r need the value rows; the value-gradient atomics need only g_r and the
// tap weights. So the two use different lane layouts: for the dots, DV = D / V lanes hold V consecutive channels
// each and one load instruction fetches 64 / DV corner rows (16 at D = 32 in 16 bits, against 2 with one channel
// per lane); for the atomics, lane `sub` holds channel sub, so an atomic instruction adds whole 128-byte lines.
// Per row: taps into LDS (lane j: sample j); every corner's value row loaded at once and dotted with g_r, the dots
// into LDS; location and weight gradients (lane j: sample j); then the atomics, which no load follows.
template <typename T, int V>
__global__ __launch_bounds__(256) void sample_backward_vec_kernel(BackParams p) {
    using A = float;
    using IO = VecIO<T, V>;
    constexpr int MAXB = 4 * kMaxLevelPoints;  // corners per row at most
    __shared__ BTap<A> taps[4][kMaxLevelPoints];
    __shared__ A dots[4][MAXB];
    const Geom& g = p.g;
    const int wv = static_cast<int>(threadIdx.x) >> 6;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wv;
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
    if (row >= rows) return;  // uniform across the wavefront; no workgroup barrier below
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int D = g.D, HD = g.H * g.D, LP = g.LP, S = 4 * LP;
    const int DV = D / V, CPI = kWave / DV;  // lanes per corner row, corners per load instruction
    const int h = static_cast<int>(row % g.H);
    const int64_t bq = row / g.H, b = bq / g.Q;
    BTap<A>* tw = taps[wv];
    A* dd = dots[wv];
    const T* __restrict__ go = static_cast<const T*>(p.grad_out) + bq * HD + h * D;

    if (lane < LP) {
        const int64_t idx = row * LP + lane;
        A lx, ly, a;
        sample_input<T, A>(p, idx, lx, ly, a);
        const int l = level_of(g, lane);
        const Taps<A> t = taps_at<A>(lx, ly, l, g, row);
        BTap<A> bt;
#pragma unroll
        for (int k = 0; k < 4; ++k) bt.tok[k] = t.tok[k];
        bt.fx = t.fx;
        bt.fy = t.fy;
        bt.a = a;
        bt.wl = static_cast<A>(g.shapes[2 * l + 1]);
        bt.hl = static_cast<A>(g.shapes[2 * l]);
        tw[lane] = bt;
    }
    __builtin_amdgcn_wave_barrier();  // LDS operations of one wavefront complete in order

    // dots: lane (corner slot cs, chunk ch) loads V channels of corner i * CPI + cs
    {
        const int cs = lane / DV, ch = lane - cs * DV;
        A gc[V];
        IO::unpack(IO::load(go + ch * V), gc);
        const T* __restrict__ vb = static_cast<const T*>(p.value) + b * g.N * HD + h * D + ch * V;
        constexpr int NB = 16;  // load instructions in flight per lane
        const int nb = (S + CPI - 1) / CPI;
        for (int i0 = 0; i0 < nb; i0 += NB) {
            typename IO::raw_t raw[NB];
            int tks[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int c = (i0 + u) * CPI + cs;
                tks[u] = i0 + u < nb && c < S ? tw[c >> 2].tok[c & 3] : -1;
                raw[u] = IO::load(vb + static_cast<int64_t>(tks[u] < 0 ? 0 : tks[u]) * HD);
            }
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int c = (i0 + u) * CPI + cs;
                A v[V];
                IO::unpack(raw[u], v);
                A d = 0;
#pragma unroll
                for (int e = 0; e < V; ++e) d += v[e] * gc[e];
                for (int m = 1; m < DV; m <<= 1) d = xor_sum(d, m);
                if (ch == 0 && i0 + u < nb && c < S) dd[c] = tks[u] >= 0 ? d : static_cast<A>(0);
            }
        }
    }
    __builtin_amdgcn_wave_barrier();

    if (lane < LP) {
        const BTap<A> bt = tw[lane];
        A d[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) d[k] = dd[4 * lane + k];
        Taps<A> t;
#pragma unroll
        for (int k = 0; k < 4; ++k) t.tok[k] = bt.tok[k];
        t.fx = bt.fx;
        t.fy = bt.fy;
        const int64_t idx = row * LP + lane;
        A ga, gx = 0, gy = 0;
        if (g.discrete) {
            ga = d[0];
        } else {
            ga = 0;
#pragma unroll
            for (int k = 0; k < 4; ++k) ga += tap_weight(t, k) * d[k];
            const A one = 1;
            const A dvx = (one - t.fy) * (d[1] - d[0]) + t.fy * (d[3] - d[2]);
            const A dvy = (one - t.fx) * (d[2] - d[0]) + t.fx * (d[3] - d[1]);
            gx = bt.a * dvx * bt.wl;
            gy = bt.a * dvy * bt.hl;
        }
        if (g.loc_acc) {
            static_cast<A*>(p.grad_loc)[2 * idx] = gx;
            static_cast<A*>(p.grad_loc)[2 * idx + 1] = gy;
            static_cast<A*>(p.grad_attn)[idx] = ga;
        } else {
            static_cast<T*>(p.grad_loc)[2 * idx] = static_cast<T>(gx);
            static_cast<T*>(p.grad_loc)[2 * idx + 1] = static_cast<T>(gy);
            static_cast<T*>(p.grad_attn)[idx] = static_cast<T>(ga);
        }
    }

    // value-gradient atomics: LG lanes per sample (LG = D rounded up to a power of two), lane sub adds channel sub
    if (p.scatter) {
        const int LG = p.LG, per = kWave / LG, slot = lane / LG, sub = lane - slot * LG;
        if (sub >= D) return;
        const A gr = cvt<A>(go[sub]);
        A* __restrict__ gv = static_cast<A*>(p.grad_value) + b * g.N * HD + h * D + sub;
        for (int j = slot; j < LP; j += per) {
            const BTap<A> bt = tw[j];
            Taps<A> t;
#pragma unroll
            for (int k = 0; k < 4; ++k) t.tok[k] = bt.tok[k];
            t.fx = bt.fx;
            t.fy = bt.fy;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int tk = bt.tok[k];
                if (tk < 0) continue;
                const A w = g.discrete ? (k == 0 ? static_cast<A>(1) : static_cast<A>(0)) : tap_weight(t, k);
                atomic_add(gv + static_cast<int64_t>(tk) * HD, bt.a * w * gr);
            }
        }
    }
}

// Sums of v[0..NB) over the n consecutive lanes of an aligned group (n = 1, 2, 4, 8 or 16; uniform), every lane of
// the group receiving them, by DPP moves within rows of 16 lanes: quad exchanges (lane ^ 1, lane ^ 2), then the
// half-row and row mirrors, which pair each lane with one of the other quad or octet, all of whose lanes hold that
// group's sums.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}
template <int NB>
__device__ __forceinline__ void group_sums(float (&v)[NB], int n) {
    if (n > 1) {
#pragma unroll
        for (int u = 0; u < NB; ++u) v[u] += dpp_mov<0xb1>(v[u]);  // quad_perm [1, 0, 3, 2]
    }
    if (n > 2) {
#pragma unroll
        for (int u = 0; u < NB; ++u) v[u] += dpp_mov<0x4e>(v[u]);  // quad_perm [2, 3, 0, 1]
    }
    if (n > 4) {
#pragma unroll
        for (int u = 0; u < NB; ++u) v[u] += dpp_mov<0x141>(v[u]);  // row_half_mirror
    }
    if (n > 8) {
#pragma unroll
        for (int u = 0; u < NB; ++u) v[u] += dpp_mov<0x140>(v[u]);  // row_mirror
    }
}

// The location and attention-weight gradients alone, for the value gradient's bucketed scatter
// (scatter_bucket_kernel), laid out like the forward sampler (td_sample.hip) rather than one row per wavefront.
// A workgroup takes RB rows, in (b, h, q) order, so that the workgroups of an XCD work through one or two heads of one
// image:
//   * taps: thread (row r, sample j) computes the sample's taps, writes its four corners' byte offsets in the value
//     buffer into LDS (kOutside when outside) and keeps the fractional position and weight in registers;
//   * dots: lane (r, corner group sg, chunk ch of V channels) loads V channels of corners sg, sg + SG, ... of row r by
//     raw buffer loads (an outside corner's load returns zeros), NB in flight, dots them with its chunk of grad_out
//     and sums the DV = D / V chunks of a corner across lanes (group_sums); d_c = value[t_c] . g_r into LDS;
//   * thread (r, j) turns its four d_c into the gradients, as sample_backward_vec_kernel does.
// Needs 16- or 32-bit types, D / V a power of two up to 16, value under 2 GB and B * Q * H * L * P below 2^31.
struct LocAttnParams {
    BackParams p;
    int RB, SG, blocks, per_xcd, val_bytes;
    FastDiv d_lp, d_gs, d_dv, d_q, d_h;  // divisions by L * P, DV * SG, DV, Q and H
};

// LDS of loc_attn_backward_body: corner byte offsets and dots, [RB][S] each (RB * LP <= 256)
constexpr size_t kLocAttnLds = 2 * 4 * 256 * sizeof(int);

// Workgroup `wg` of loc_attn_backward_kernel's grid, with `lds` its kLocAttnLds bytes (16-byte aligned).
template <typename T, int V, int NB>
__device__ __forceinline__ void loc_attn_backward_body(const LocAttnParams& lp, int wg, unsigned char* lds) {
    constexpr int NTH = 256;
    using A = float;
    using IO = VecIO<T, V>;
    using R = typename IO::raw_t;
    const BackParams& p = lp.p;
    const Geom& g = p.g;
    const int LP = g.LP, S = 4 * LP, D = g.D, HD = g.H * D, DV = D / V, SG = lp.SG, GS = DV * SG, RB = lp.RB;
    int* off = reinterpret_cast<int*>(lds);             // [RB][S] corner byte offsets (RB * LP <= NTH)
    A* dots = reinterpret_cast<A*>(lds) + 4 * NTH;      // [RB][S] value row . grad_out row
    const int tid = threadIdx.x;
    const int blk = (wg % kXcds) * lp.per_xcd + wg / kXcds;
    if (blk >= lp.blocks) return;  // the whole workgroup
    const int rows = g.B * g.Q * g.H, i0 = blk * RB;
    // row (b, q, h) of the i-th row in (b, h, q) order
    const auto row_of = [&](int i, int& b, int& h) {
        const int bh = static_cast<int>(fast_div(lp.d_q, static_cast<uint32_t>(i))), q = i - bh * g.Q;
        b = static_cast<int>(fast_div(lp.d_h, static_cast<uint32_t>(bh)));
        h = bh - b * g.H;
        return (b * g.Q + q) * g.H + h;
    };

    const int sb = HD * static_cast<int>(sizeof(T));
    A fx = 0, fy = 0, a = 0, wl = 0, hl = 0;
    int64_t idx = -1;  // this thread's sample, -1 for none
    int rs = 0, js = 0;
    if (tid < RB * LP) {
        rs = static_cast<int>(fast_div(lp.d_lp, static_cast<uint32_t>(tid)));
        js = tid - rs * LP;
        int* o4 = off + rs * S + 4 * js;
        if (i0 + rs < rows) {
            int b, h;
            const int row = row_of(i0 + rs, b, h);
            idx = static_cast<int64_t>(row) * LP + js;
            A lx, ly;
            sample_input<T, A>(p, idx, lx, ly, a);
            const int l = level_of(g, js);
            const Taps<A> t = taps_at_b<A>(lx, ly, l, g, b);
#pragma unroll
            for (int k = 0; k < 4; ++k) o4[k] = t.tok[k] >= 0 ? t.tok[k] * sb : kOutside;
            fx = t.fx;
            fy = t.fy;
            wl = static_cast<A>(g.shapes[2 * l + 1]);
            hl = static_cast<A>(g.shapes[2 * l]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) o4[k] = kOutside;
        }
    }
    __syncthreads();

    const __amdgpu_buffer_rsrc_t rsrc = buffer_of(p.value, lp.val_bytes);
    const T* __restrict__ go = static_cast<const T*>(p.grad_out);
    for (int it = tid; it < RB * GS; it += NTH) {
        const int r = static_cast<int>(fast_div(lp.d_gs, static_cast<uint32_t>(it))), rem = it - r * GS;
        const int sg = static_cast<int>(fast_div(lp.d_dv, static_cast<uint32_t>(rem))), ch = rem - sg * DV;
        int b = 0, h = 0, row = 0;
        const bool valid = i0 + r < rows;
        if (valid) row = row_of(i0 + r, b, h);
        A gc[V];
        IO::unpack(valid ? IO::load(go + static_cast<int64_t>(row) * D + ch * V) : IO::zero(), gc);
        const unsigned lane_off =
            static_cast<unsigned>((static_cast<int64_t>(b) * g.N * HD + h * D + ch * V) * static_cast<int>(sizeof(T)));
        const int* __restrict__ orow = off + r * S;
        A* __restrict__ drow = dots + r * S;
        for (int s0 = sg; s0 < S; s0 += SG * NB) {
            R raw[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                const int s = s0 + u * SG;
                raw[u] = buffer_load<R>(rsrc, static_cast<unsigned>(s < S ? orow[s] : kOutside) + lane_off);
            }
            A d[NB];
#pragma unroll
            for (int u = 0; u < NB; ++u) {
                A v[V];
                IO::unpack(raw[u], v);
                d[u] = 0;
#pragma unroll
                for (int e = 0; e < V; ++e) d[u] = fmaf(v[e], gc[e], d[u]);
            }
            group_sums(d, DV);
            if (ch == 0) {
#pragma unroll
                for (int u = 0; u < NB; ++u)
                    if (s0 + u * SG < S) drow[s0 + u * SG] = d[u];
            }
        }
    }
    __syncthreads();

    if (idx >= 0) {
        A d[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) d[k] = dots[rs * S + 4 * js + k];
        A ga, gx = 0, gy = 0;
        if (g.discrete) {
            ga = d[0];
        } else {
            const A one = 1;
            ga = (one - fx) * (one - fy) * d[0] + fx * (one - fy) * d[1] + (one - fx) * fy * d[2] + fx * fy * d[3];
            const A dvx = (one - fy) * (d[1] - d[0]) + fy * (d[3] - d[2]);
            const A dvy = (one - fx) * (d[2] - d[0]) + fx * (d[3] - d[1]);
            gx = a * dvx * wl;
            gy = a * dvy * hl;
        }
        if (g.loc_acc) {
            static_cast<A*>(p.grad_loc)[2 * idx] = gx;
            static_cast<A*>(p.grad_loc)[2 * idx + 1] = gy;
            static_cast<A*>(p.grad_attn)[idx] = ga;
        } else {
            static_cast<T*>(p.grad_loc)[2 * idx] = static_cast<T>(gx);
            static_cast<T*>(p.grad_loc)[2 * idx + 1] = static_cast<T>(gy);
            static_cast<T*>(p.grad_attn)[idx] = static_cast<T>(ga);
        }
    }
}

template <typename T, int V, int NB>
__global__ __launch_bounds__(256) void loc_attn_backward_kernel(LocAttnParams lp) {
    __shared__ __align__(16) unsigned char lds[kLocAttnLds];
    loc_attn_backward_body<T, V, NB>(lp, static_cast<int>(blockIdx.x), lds);
}

// The value-gradient scatter where many queries sample the same neighbourhood (encoder self-attention: every token
// a query, sampling a few pixels around itself on every level). The scatter is bound by the float atomics, at a
// rate per 128-byte line; consecutive queries of one head touch overlapping pixels (16 of them about 2.4 times fewer
// pixels than corners on DINO-style encoder inputs), so their corners are summed per pixel first and each touched
// pixel goes out once. Workgroup = (image b, head h, QT consecutive queries), one (row, sample) per thread; per level:
//   * the bounding box of the level's in-map corners (wavefront min / max by DPP, then over the wavefronts in LDS;
//     the boxes of up to 8 levels are found together, behind one barrier);
//   * if it holds at most kBucketPix pixels: a counting sort of the corners by pixel (an integer LDS atomic per corner
//     gives its rank in the pixel's bucket; a workgroup scan of the counts gives each bucket's start and the list
//     of touched pixels with their buckets' start, count and token); then D lanes per touched pixel sum its
//     bucket's a * w_c * g_r from LDS, without atomics, and add the sums to grad_value (one D-wide atomic per channel
//     group). A bucket entry holds its coefficient and grad_out row itself, so a sum reads two LDS values per entry,
//     one after the other (the entry, then the row's channel);
//   * otherwise the level's corners are added to grad_value directly, as sample_backward_vec_kernel does.
// Five barriers per bucketed level: the ranks, the scan's wavefront totals, the bucket starts, the list, the sums
// (the counts are cleared during the sums for the next level).
// D is a power of two from 4 to 64 (lane = channel tid % D), P > 0. The sums reach grad_value in another order than
// the direct scatter's, so the two agree to float rounding.
constexpr int kBucketPix = 1024;  // bounding-box pixels per level at most
constexpr int kTileW = 8, kTileH = 4;  // self-attention tiles: 8 x 4 pixels of a level's map (QT = 32 queries)
constexpr int kBucketEnt = 1024;  // corner entries per level at most: QT * P * 4 with QT * L * P <= 256

// a bucketed corner: its coefficient a * w_c and the offset of its grad_out row in LDS (r * D)
struct alignas(8) BucketEntry {
    float coef;
    int row;
};

struct BucketParams {
    const void* loc;
    const void* attn;
    const void* grad_out;
    void* grad_value;  // [B, N, H * D] float, zeroed
    Geom g;
    int QT, qtiles, units, per_xcd;
    FastDiv d_lp, d_p;  // divisions by L * P and P
};

// Reductions over the 64 lanes of a wavefront by DPP moves within rows of 16 lanes (every lane of a row then holds
// the row's result) and reads of lanes 0, 16, 32 and 48: no LDS round trips. All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int x) {
    return __builtin_amdgcn_mov_dpp(x, CTRL, 0xf, 0xf, false);
}
__device__ __forceinline__ int wave_min(int v) {
    v = min(v, dpp_mov_i<0xb1>(v));   // quad_perm [1, 0, 3, 2]
    v = min(v, dpp_mov_i<0x4e>(v));   // quad_perm [2, 3, 0, 1]
    v = min(v, dpp_mov_i<0x141>(v));  // row_half_mirror
    v = min(v, dpp_mov_i<0x140>(v));  // row_mirror
    return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}
__device__ __forceinline__ int wave_max(int v) {
    v = max(v, dpp_mov_i<0xb1>(v));
    v = max(v, dpp_mov_i<0x4e>(v));
    v = max(v, dpp_mov_i<0x141>(v));
    v = max(v, dpp_mov_i<0x140>(v));
    return max(max(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
               max(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Inclusive prefix sum over the 64 lanes of a wavefront: within each row by adds of the row shifted right by 1, 2, 4
// and 8 lanes (lanes shifted in from outside the row read 0), then each row plus the totals of the rows before it.
// All 64 lanes must be active.
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31);
    const int r2 = __builtin_amdgcn_readlane(v, 47), row = lane_id() >> 4;
    return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

template <typename T, int NTH, bool TILE2D>
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(6))) void scatter_bucket_kernel(BucketParams bp) {
    using A = float;
    constexpr int NW = NTH / kWave;
    constexpr int LB = 8;  // levels whose bounding boxes are found together
    const Geom& g = bp.g;
    const int D = g.D, HD = g.H * g.D, LP = g.LP, P = g.P, QT = bp.QT;
    const int tid = threadIdx.x, d = tid & (D - 1), grp = tid / D, ngrp = NTH / D;
    const int wave = tid >> 6, lane = tid & (kWave - 1);

    __shared__ A gr[2 * NTH];                 // [QT][D] (QT * D <= 2 * NTH)
    __shared__ int etok[kBucketEnt];          // direct levels: corner token, -1 outside
    __shared__ A ecoef[kBucketEnt];           // a * w_c
    __shared__ int erow[kBucketEnt];          // the corner's row offset in gr (r * D)
    __shared__ int cnt[kBucketPix];           // corners per window pixel (zero between levels)
    __shared__ int base[kBucketPix];          // start of the pixel's bucket in lent
    __shared__ int2 tinfo[kBucketEnt];        // touched pixels (compacted): bucket start | count << 16, token
    __shared__ BucketEntry lent[kBucketEnt];  // entries bucketed by pixel: a * w_c and grad_out row offset
    __shared__ int boxw[LB][NW][4];           // per level and wavefront: min x, min y, max x, max y
    __shared__ int wtot[NW];

    const T* __restrict__ go = static_cast<const T*>(bp.grad_out);
    for (int i = tid; i < kBucketPix; i += NTH) cnt[i] = 0;

    // One tile: rows r < QT of image b and head h, row r being query query_of(r) (-1: no query; its samples have
    // no corner in the map)
    auto tile = [&](int b, int h, auto query_of) {
        A* __restrict__ gv =
            static_cast<A*>(bp.grad_value) + static_cast<int64_t>(b) * g.N * HD + static_cast<int64_t>(h) * D;
        for (int i = tid; i < QT * D; i += NTH) {
            const int r = i / D, q = query_of(r);
            gr[i] = q >= 0 ? cvt<A>(go[(static_cast<int64_t>(b) * g.Q + q) * HD + static_cast<int64_t>(h) * D +
                                       (i - r * D)])
                           : static_cast<A>(0);
        }

        // this thread's sample (row r, sample j of level lt): its four corners' tokens, pixels and coefficients
        int tk[4] = {-1, -1, -1, -1}, cx[4] = {0, 0, 0, 0}, cy[4] = {0, 0, 0, 0};
        A cf[4] = {0, 0, 0, 0};
        int lt = -1, r = 0, jp = 0;
        if (tid < QT * LP) {
            r = static_cast<int>(fast_div(bp.d_lp, static_cast<uint32_t>(tid)));
            const int j = tid - r * LP;
            lt = static_cast<int>(fast_div(bp.d_p, static_cast<uint32_t>(j)));
            jp = j - lt * P;
            const int q = query_of(r);
            if (q >= 0) {
                const int64_t row = (static_cast<int64_t>(b) * g.Q + q) * g.H + h, idx = row * LP + j;
                A lx, ly, a;
                if (g.loc_acc) {
                    lx = static_cast<const A*>(bp.loc)[2 * idx];
                    ly = static_cast<const A*>(bp.loc)[2 * idx + 1];
                    a = static_cast<const A*>(bp.attn)[idx];
                } else {
                    lx = cvt<A>(static_cast<const T*>(bp.loc)[2 * idx]);
                    ly = cvt<A>(static_cast<const T*>(bp.loc)[2 * idx + 1]);
                    a = cvt<A>(static_cast<const T*>(bp.attn)[idx]);
                }
                const Taps<A> t = taps_at_b<A>(lx, ly, lt, g, b);
                const int wl = static_cast<int>(g.shapes[2 * lt + 1]);
                const int64_t st = g.starts[lt];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    tk[k] = t.tok[k];
                    cf[k] = g.discrete ? (k == 0 ? a : static_cast<A>(0)) : a * tap_weight(t, k);
                    if (tk[k] >= 0) {
                        const int loc = static_cast<int>(tk[k] - st);
                        cy[k] = loc / wl;
                        cx[k] = loc - cy[k] * wl;
                    }
                }
            }
        }

        for (int l = 0; l < g.L; ++l) {
            if (l % LB == 0) {
                // bounding boxes of the in-map corners of levels l .. l + LB - 1, per wavefront
                if (l > 0) __syncthreads();  // every wavefront has read the previous group's boxes
                for (int ll = l; ll < g.L && ll < l + LB; ++ll) {
                    int mnx = 0x7fffffff, mny = 0x7fffffff, mxx = -1, mxy = -1;
                    if (lt == ll) {
#pragma unroll
                        for (int k = 0; k < 4; ++k)
                            if (tk[k] >= 0) {
                                mnx = min(mnx, cx[k]);
                                mny = min(mny, cy[k]);
                                mxx = max(mxx, cx[k]);
                                mxy = max(mxy, cy[k]);
                            }
                    }
                    mnx = wave_min(mnx);
                    mny = wave_min(mny);
                    mxx = wave_max(mxx);
                    mxy = wave_max(mxy);
                    if (lane == 0) {
                        boxw[ll - l][wave][0] = mnx;
                        boxw[ll - l][wave][1] = mny;
                        boxw[ll - l][wave][2] = mxx;
                        boxw[ll - l][wave][3] = mxy;
                    }
                }
                __syncthreads();  // the boxes (and, first, the grad_out rows and the zeroed counts) are in place
            }
            const int lb = l % LB;
            int x0 = boxw[lb][0][0], y0 = boxw[lb][0][1], x1 = boxw[lb][0][2], y1 = boxw[lb][0][3];
#pragma unroll
            for (int w = 1; w < NW; ++w) {
                x0 = min(x0, boxw[lb][w][0]);
                y0 = min(y0, boxw[lb][w][1]);
                x1 = max(x1, boxw[lb][w][2]);
                y1 = max(y1, boxw[lb][w][3]);
            }
            if (x1 < x0) continue;  // no in-map corner on this level (uniform)
            const bool mine = lt == l;
            const int bw = x1 - x0 + 1;
            const int64_t npix64 = static_cast<int64_t>(bw) * (y1 - y0 + 1);
            if (npix64 <= kBucketPix) {
                const int npix = static_cast<int>(npix64);
                const int wl = static_cast<int>(g.shapes[2 * l + 1]);
                const int64_t st = g.starts[l];
                int px[4], rank[4];
                if (mine) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        px[k] = (cy[k] - y0) * bw + (cx[k] - x0);
                        rank[k] = tk[k] >= 0 ? atomicAdd(&cnt[px[k]], 1) : 0;
                    }
                }
                __syncthreads();
                // workgroup scan of the counts: thread t owns pixels [t * k, t * k + k), k = ceil(npix / NTH);
                // packed (touched pixels << 16) | corners
                const int kp = (npix + NTH - 1) / NTH, p0 = tid * kp;
                int own = 0;
                for (int i = 0; i < kp; ++i) {
                    const int pp = p0 + i;
                    const int c = pp < npix ? cnt[pp] : 0;
                    own += c + (c > 0 ? (1 << 16) : 0);
                }
                const int incl = wave_incl_scan(own);
                if (lane == kWave - 1) wtot[wave] = incl;
                __syncthreads();
                int before = 0;
                for (int w = 0; w < wave; ++w) before += wtot[w];
                int total = 0;
#pragma unroll
                for (int w = 0; w < NW; ++w) total += wtot[w];
                int run = before + incl - own;  // exclusive
                for (int i = 0; i < kp; ++i) {
                    const int pp = p0 + i;
                    if (pp >= npix) break;
                    const int c = cnt[pp];
                    base[pp] = run & 0xffff;
                    if (c > 0) {
                        const int yy = pp / bw;
                        tinfo[run >> 16] = make_int2((run & 0xffff) | c << 16,
                                                     static_cast<int>(st + static_cast<int64_t>(y0 + yy) * wl +
                                                                      (x0 + pp - yy * bw)));
                    }
                    run += c + (c > 0 ? (1 << 16) : 0);
                }
                __syncthreads();
                if (mine) {
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (tk[k] >= 0) lent[base[px[k]] + rank[k]] = BucketEntry{cf[k], r * D};
                }
                __syncthreads();
                // the counts are no longer read (the touched pixels carry theirs): cleared for the next level
                for (int i = tid; i < npix; i += NTH) cnt[i] = 0;
                const int ntouched = total >> 16;
                for (int ti = grp; ti < ntouched; ti += ngrp) {
                    const int2 info = tinfo[ti];
                    const int s0 = info.x & 0xffff, n = info.x >> 16;
                    A v = 0;
                    int i = 0;
                    for (; i + 1 < n; i += 2) {  // two entries' reads in flight
                        const BucketEntry u = lent[s0 + i], w = lent[s0 + i + 1];
                        const A gu = gr[u.row + d], gw = gr[w.row + d];
                        v += u.coef * gu;
                        v += w.coef * gw;
                    }
                    if (i < n) {
                        const BucketEntry u = lent[s0 + i];
                        v += u.coef * gr[u.row + d];
                    }
                    atomic_add(gv + static_cast<int64_t>(info.y) * HD + d, v);
                }
                __syncthreads();  // the counts are zero and the buckets free for the next level
            } else {
                if (mine) {
                    const int e0 = (r * P + jp) * 4;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        etok[e0 + k] = tk[k];
                        ecoef[e0 + k] = cf[k];
                        erow[e0 + k] = r * D;
                    }
                }
                __syncthreads();
                const int ne = QT * P * 4;  // the level's corner entries (rows without a query: none in the map)
                for (int e = grp; e < ne; e += ngrp) {
                    const int t = etok[e];
                    if (t >= 0) atomic_add(gv + static_cast<int64_t>(t) * HD + d, ecoef[e] * gr[erow[e] + d]);
                }
                __syncthreads();  // the entries are free for the next level
            }
        }
    };

    if constexpr (!TILE2D) {
        // QT consecutive queries
        const int unit = (blockIdx.x % kXcds) * bp.per_xcd + blockIdx.x / kXcds;
        if (unit >= bp.units) return;  // the whole workgroup
        const int qt = unit % bp.qtiles, bh = unit / bp.qtiles;
        const int q0 = qt * QT, nq = g.Q - q0 < QT ? g.Q - q0 : QT;
        tile(bh / g.H, bh % g.H, [&](int r) { return r < nq ? q0 + r : -1; });
    } else {
        // self-attention (Q = N, query q at token q's pixel): tiles of kTileW x kTileH pixels of each level's map, in
        // level order; the level sizes are on the device, so every workgroup counts the tiles and takes every
        // gridDim.x-th
        auto level_tiles = [&](int l, int& nbx) {
            const int wl = static_cast<int>(g.shapes[2 * l + 1]), hl = static_cast<int>(g.shapes[2 * l]);
            nbx = (wl + kTileW - 1) / kTileW;
            return nbx * ((hl + kTileH - 1) / kTileH);
        };
        int per_bh = 0;
        for (int l = 0; l < g.L; ++l) {
            int nbx;
            per_bh += level_tiles(l, nbx);
        }
        const int tiles = g.B * g.H * per_bh;
        for (int t = blockIdx.x; t < tiles; t += gridDim.x) {
            __syncthreads();  // every wavefront is done with the previous tile's LDS
            const int bh = t / per_bh;
            int rest = t - bh * per_bh, lq = 0, nbx = 1;
            for (; lq < g.L; ++lq) {
                const int n = level_tiles(lq, nbx);
                if (rest < n) break;
                rest -= n;
            }
            const int wl = static_cast<int>(g.shapes[2 * lq + 1]), hl = static_cast<int>(g.shapes[2 * lq]);
            const int x0 = (rest % nbx) * kTileW, y0 = (rest / nbx) * kTileH;
            const int st = static_cast<int>(g.starts[lq]);
            tile(bh / g.H, bh % g.H, [&](int r) {
                const int x = x0 + r % kTileW, y = y0 + r / kTileW;
                return x < wl && y < hl ? st + y * wl + x : -1;
            });
        }
    }
}

// The value gradient by binning the corners by token (decoder shapes, 16-bit types). With few corner hits per token
// (decoders: 2-4 per token and head) the atomic scatter runs at the GPU's float-atomic rate (about 320 G lane-adds/s,
// one 128-byte line per corner at D = 32) and needs a zeroed float32 accumulator and a rounding pass. LDS float
// atomics are no way out: ds_add_f32 runs at about 0.33 lanes per clock per CU (about 200 G lane-adds/s over the GPU,
// whatever the bank pattern), against about 13 for integer LDS atomics. Instead, per (image b, head h):
//   * bins: level l's tokens go in bins of 2^shift_l consecutive tokens, the widest power of two from the minimum
//     (8 or more, chosen on the host so that the bins fit) to TB (128; 64 at D = 64) whose bin expects at most
//     kSortTarget entries (4 Q P_l corners over the level's n_l tokens): the small, densely sampled levels get narrow
//     bins (sort_levels, from the device-resident level shapes);
//   * sort_count_kernel: each query tile counts its corners into the bins (LDS counters);
//   * sort_scan_body (in scan_loc_attn_kernel, beside the location and weight gradients): one workgroup per (b, h)
//     scans the counts, bin-major, into each tile's start within each bin and each bin's start; then it lists the
//     reduce items: one per bin, or, for a bin above kSortChunk entries (a hot spot), 2^j token ranges, the fewest
//     averaging at most kSortChunk entries each;
//   * sort_fill_kernel: each tile writes its corners as entries {a * w_c, row << 7 | position in the bin} into their
//     bins (ranks within the tile from LDS atomics);
//   * sort_reduce_kernel: one workgroup per item reads its bin's entries kSortChunk at a time and sorts those of its
//     range in LDS (a counting sort: integer LDS atomics for the ranks) so that each lane group's tokens' entries lie
//     together; each group then streams through its entries, 8 grad_out rows in flight per lane, adding the products
//     a * w_c * g_row into its own tokens' float sums in LDS; finally the workgroup writes its tokens' rows, in the
//     element type.
// No float atomics, no zero fill, no rounding pass. Within a token the products are added in the order the LDS ranks
// give, so the result agrees with the atomic scatter's to float rounding. The scratch (entries, items, counts,
// starts) lives in the caller's float32 accumulator buffer. grad_loc and grad_attn come from
// loc_attn_backward_kernel.
constexpr int kSortMaxBins = 8192;  // bins per (b, h) at most (the tiles' LDS counters)
constexpr int kSortChunk = 512;     // entries per token range on average at most; entries read per round
constexpr int kSortTarget = 512;    // expected entries per bin at most (where the bin can be that narrow)

// tokens per bin at most at head width D: TB x D floats = 16 KB (128 at most: an entry keeps its position in the
// bin in 7 bits)
__host__ __device__ constexpr int sort_bin_tokens(int D) { return D >= 64 ? 4096 / D : 128; }

struct SortParams {
    const void* loc;
    const void* attn;
    const void* grad_out;
    void* grad_value;  // [B, N, H * D] element type
    Geom g;
    int QT, qtiles;       // queries per tile (256 / (L * P)), tiles per (b, h)
    int nb;               // bins per (b, h) at most (the levels' bins, computed on the device, are clamped to it)
    int tb_shift;         // log2 of the tokens per bin at most
    int min_shift;        // log2 of the tokens per bin at least
    int maxch;            // reduce items per (b, h) at most
    int64_t cap;          // entries per (b, h) at most: Q * L * P * 4
    int* hist;            // [B * H][nb][qtiles]: counts, then each tile's start within its bin
    int* bin_start;       // [B * H][nb + 1]: each bin's first entry (sort_scan_body)
    uint4* items;         // [B * H * maxch]: the reduce items of every (b, h) (sort_item)
    int* counters;        // [1]: items listed (zeroed by sort_count_kernel)
    uint2* entries;       // [B * H][cap]
    FastDiv d_lp;
};

// The bins of the levels: level l's tokens start[l] .. start[l] + n[l] - 1 (clamped into [0, N)) in bins of
// 2^shift[l] tokens, numbered base[l] .. base[l + 1] - 1 (base[L] = the bins in use, at most sp.nb).
struct SortLevels {
    int base[kMaxLevelPoints + 1];
    int shift[kMaxLevelPoints];
    int start[kMaxLevelPoints];
    int n[kMaxLevelPoints];
};

// A reduce item: bin tokens t0 .. t0 + 2^shift - 1 of (b, h) = bh, of which `tokens` exist, range k of 2^j of them;
// its entries first .. end - 1 of the (b, h)'s. t0 < 2^20 (N / 2^min_shift + L bins of at most 128 tokens stay within
// kSortMaxBins), bh < 2^23 (checked on the host).
struct SortItem {
    int t0, bh, first, end, shift, j, k, tokens;
};
__host__ __device__ inline uint4 sort_item_pack(const SortItem& i) {
    return make_uint4(static_cast<unsigned>(i.t0) | static_cast<unsigned>(i.bh & 0xfff) << 20,
                      static_cast<unsigned>(i.first), static_cast<unsigned>(i.end),
                      static_cast<unsigned>(i.shift | i.j << 3 | i.k << 6 | i.tokens << 13 | (i.bh >> 12) << 21));
}
__device__ inline SortItem sort_item_unpack(const uint4& u) {
    SortItem i;
    i.t0 = static_cast<int>(u.x & 0xfffffu);
    i.bh = static_cast<int>(u.x >> 20 | (u.w >> 21) << 12);
    i.first = static_cast<int>(u.y);
    i.end = static_cast<int>(u.z);
    i.shift = static_cast<int>(u.w & 7u);
    i.j = static_cast<int>((u.w >> 3) & 7u);
    i.k = static_cast<int>((u.w >> 6) & 0x7fu);
    i.tokens = static_cast<int>((u.w >> 13) & 0xffu);
    return i;
}

// Fills lv; called by a whole wavefront (every lane active), the caller's barrier publishes it.
__device__ void sort_levels(const SortParams& sp, SortLevels& lv) {
    const Geom& g = sp.g;
    const int l = lane_id();
    int nbins = 0;
    if (l < g.L) {
        const int64_t st = g.starts[l], n64 = g.shapes[2 * l] * g.shapes[2 * l + 1];
        const int64_t s0 = st < 0 ? 0 : (st > g.N ? g.N : st);
        const int64_t n = n64 < 0 ? 0 : (n64 > g.N - s0 ? g.N - s0 : n64);
        const int pl = g.P > 0 ? g.P : g.level_end[l] - (l > 0 ? g.level_end[l - 1] : 0);
        const int64_t corners = int64_t{4} * g.Q * pl;
        int shift = sp.min_shift;
        while (shift < sp.tb_shift && (corners << (shift + 1)) <= int64_t{kSortTarget} * n) ++shift;
        nbins = static_cast<int>((n + (int64_t{1} << shift) - 1) >> shift);
        lv.shift[l] = shift;
        lv.start[l] = static_cast<int>(s0);
        lv.n[l] = static_cast<int>(n);
    }
    const int incl = wave_incl_scan(nbins);
    if (l < g.L) lv.base[l + 1] = min(incl, sp.nb);
    if (l == 0) lv.base[0] = 0;
}

// Thread tid of tile (bh, qt): its sample's four corners (tokens, -1 outside) and coefficients, its level and row.
template <typename T>
__device__ __forceinline__ bool sort_sample(const SortParams& sp, int bh, int qt, int tid, int (&tk)[4],
                                            float (&cf)[4], int& lev, int& row) {
    const Geom& g = sp.g;
    if (tid >= sp.QT * g.LP) return false;
    const int r = static_cast<int>(fast_div(sp.d_lp, static_cast<uint32_t>(tid))), j = tid - r * g.LP;
    const int q = qt * sp.QT + r;
    if (q >= g.Q) return false;
    const int b = bh / g.H, h = bh - b * g.H;
    row = (b * g.Q + q) * g.H + h;
    const int64_t idx = static_cast<int64_t>(row) * g.LP + j;
    float lx, ly, a;
    if (g.loc_acc) {
        lx = static_cast<const float*>(sp.loc)[2 * idx];
        ly = static_cast<const float*>(sp.loc)[2 * idx + 1];
        a = static_cast<const float*>(sp.attn)[idx];
    } else {
        lx = cvt<float>(static_cast<const T*>(sp.loc)[2 * idx]);
        ly = cvt<float>(static_cast<const T*>(sp.loc)[2 * idx + 1]);
        a = cvt<float>(static_cast<const T*>(sp.attn)[idx]);
    }
    lev = level_of(g, j);
    const Taps<float> t = taps_at_b<float>(lx, ly, lev, g, b);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        tk[k] = t.tok[k];
        cf[k] = g.discrete ? (k == 0 ? a : 0.f) : a * tap_weight(t, k);
    }
    return true;
}

// The bin of token tk of level l and its position in the bin (-1 for a token outside the level's clamped range)
__device__ __forceinline__ int sort_bin_of(const SortLevels& lv, int l, int tk, int& pos) {
    const int rel = tk - lv.start[l];
    if (static_cast<unsigned>(rel) >= static_cast<unsigned>(lv.n[l])) return -1;
    const int bin = lv.base[l] + (rel >> lv.shift[l]);
    pos = rel & ((1 << lv.shift[l]) - 1);
    return bin < lv.base[l + 1] ? bin : -1;
}

template <typename T>
__global__ __launch_bounds__(256) void sort_count_kernel(SortParams sp) {
    extern __shared__ int lc[];  // [nb]
    __shared__ SortLevels lv;
    const int bh = blockIdx.x / sp.qtiles, qt = blockIdx.x - bh * sp.qtiles;
    if (blockIdx.x == 0 && threadIdx.x == 0) sp.counters[0] = 0;  // for sort_scan_body's reservations
    for (int i = threadIdx.x; i < sp.nb; i += 256) lc[i] = 0;
    int tk[4], lev, row;
    float cf[4];
    const bool has = sort_sample<T>(sp, bh, qt, threadIdx.x, tk, cf, lev, row);  // its loads overlap the table's
    if (threadIdx.x < kWave) sort_levels(sp, lv);
    __syncthreads();  // the level table and the cleared counters
    const int nb = lv.base[sp.g.L];
    if (has) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int pos;
            const int bin = tk[k] >= 0 ? sort_bin_of(lv, lev, tk[k], pos) : -1;
            if (bin >= 0) atomicAdd(&lc[bin], 1);
        }
    }
    __syncthreads();
    int* hist = sp.hist + static_cast<int64_t>(bh) * sp.nb * sp.qtiles;
    for (int i = threadIdx.x; i < nb; i += 256) hist[static_cast<int64_t>(i) * sp.qtiles + qt] = lc[i];
}

// One workgroup per (b, h). First the exclusive scan of the nb * qtiles counts (bin-major) in chunks of 4096, each
// loaded into LDS with coalesced reads, thread t owning 8 consecutive counts (LDS pitch 9 words: the owners' reads
// spread over the banks), a wavefront scan of the owners' totals, and coalesced writes back; the bins' starts are the
// scanned values at the bins' first counts (kept in LDS, bst). Then the reduce items of the (b, h)'s bins.
constexpr int kScanTh = 256, kScanK = 8, kScanChunk = kScanTh * kScanK;

__device__ __forceinline__ int block_excl_scan(int x, int* wt, int wave, int lane, int& total) {
    constexpr int NW = kScanTh / kWave;
    const int incl = wave_incl_scan(x);  // every lane active
    if (lane == kWave - 1) wt[wave] = incl;
    __syncthreads();
    int run = incl - x, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        run += w < wave ? wt[w] : 0;
        tot += wt[w];
    }
    total = tot;
    return run;
}

// LDS of sort_scan_body: the chunk (pitch kScanK + 1), the wavefront totals, the place in the item list, the level
// table
constexpr size_t kScanV = static_cast<size_t>(kScanTh) * (kScanK + 1) * sizeof(int);
constexpr size_t kScanLds = kScanV + (kScanTh / kWave + 4) * sizeof(int) + sizeof(SortLevels);

// Workgroup of (b, h) = bh, with `lds` its kScanLds bytes (16-byte aligned).
__device__ __forceinline__ void sort_scan_body(const SortParams& sp, int bh, unsigned char* lds) {
    int* v = reinterpret_cast<int*>(lds);
    int* wtot = reinterpret_cast<int*>(lds + kScanV);
    int& place = wtot[kScanTh / kWave];
    SortLevels& lv = *reinterpret_cast<SortLevels*>(lds + kScanV + (kScanTh / kWave + 4) * sizeof(int));
    int* bst = sp.bin_start + static_cast<int64_t>(bh) * (sp.nb + 1);  // the bins' starts (read back after a barrier)
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & (kWave - 1);
    if (tid < kWave) sort_levels(sp, lv);
    __syncthreads();
    const int nb = lv.base[sp.g.L];
    int* hist = sp.hist + static_cast<int64_t>(bh) * sp.nb * sp.qtiles;
    const int n = nb * sp.qtiles;  // < 2^30 (checked on the host)
    int* mine = v + tid * (kScanK + 1);
    int carry = 0;
    int hv[kScanK];  // a chunk's counts, loaded at clamped indexes (all in flight together) a chunk ahead
    if (n > 0) {
#pragma unroll
        for (int u = 0; u < kScanK; ++u) hv[u] = hist[min(tid + u * kScanTh, min(n, kScanChunk) - 1)];
    }
    for (int c0 = 0; c0 < n; c0 += kScanChunk) {  // uniform: every barrier is reached by the whole workgroup
        const int len = n - c0 < kScanChunk ? n - c0 : kScanChunk;
#pragma unroll
        for (int u = 0; u < kScanK; ++u) {
            const int j = tid + u * kScanTh;
            v[(j / kScanK) * (kScanK + 1) + j % kScanK] = j < len ? hv[u] : 0;
        }
        // the next chunk's counts (no branch, so that the loads stay in flight: past the end they reread the last
        // count, unused)
#pragma unroll
        for (int u = 0; u < kScanK; ++u) hv[u] = hist[min(c0 + kScanChunk + tid + u * kScanTh, n - 1)];
        __syncthreads();  // the chunk is in LDS
        int own = 0;
#pragma unroll
        for (int k = 0; k < kScanK; ++k) own += mine[k];
        int tot;
        int run = carry + block_excl_scan(own, wtot, wave, lane, tot);
#pragma unroll
        for (int k = 0; k < kScanK; ++k) {
            const int c = mine[k];
            mine[k] = run;
            run += c;
        }
        __syncthreads();  // the chunk is scanned
        for (int j = tid; j < len; j += kScanTh) hist[c0 + j] = v[(j / kScanK) * (kScanK + 1) + j % kScanK];
        // bins whose first count lies in this chunk
        for (int bb = (c0 + sp.qtiles - 1) / sp.qtiles + tid; static_cast<int64_t>(bb) * sp.qtiles < c0 + len;
             bb += kScanTh) {
            const int j = bb * sp.qtiles - c0;
            bst[bb] = v[(j / kScanK) * (kScanK + 1) + j % kScanK];
        }
        carry += tot;
        __syncthreads();  // v and wtot are free for the next chunk
    }
    if (tid == 0) bst[nb] = carry;
    __syncthreads();  // every bin's start is in bst
    // the items: one per bin, or 2^lj token ranges of a bin above kSortChunk entries (the fewest averaging at most
    // kSortChunk entries each), the split ones first (they read several rounds of entries: the longest); the (b, h)
    // reserves its places in the list with one atomic
    auto level_of_bin = [&](int bin) {
        int l = 0;
        while (l + 1 < sp.g.L && bin >= lv.base[l + 1]) ++l;
        return l;
    };
    auto split_of = [&](int bin, int l) {
        const int cnt = bst[bin + 1] - bst[bin];
        int lj = 0;
        while (lj < lv.shift[l] && (cnt >> lj) > kSortChunk) ++lj;
        return lj;
    };
    int own_split = 0, own_other = 0;
    for (int bin = tid; bin < nb; bin += kScanTh) {
        const int lj = split_of(bin, level_of_bin(bin));
        own_split += lj > 0 ? 1 << lj : 0;
        own_other += lj > 0 ? 0 : 1;
    }
    int tot_split, tot_other;
    block_excl_scan(own_split, wtot, wave, lane, tot_split);
    __syncthreads();  // wtot is free
    block_excl_scan(own_other, wtot, wave, lane, tot_other);
    if (tid == 0) place = atomicAdd(sp.counters, tot_split + tot_other);
    __syncthreads();  // the place is known; wtot is free
    uint4* list = sp.items + place;
    int run_split = 0, run_other = tot_split;
    for (int b0 = 0; b0 < nb; b0 += kScanTh) {  // uniform
        const int bin = b0 + tid;
        const int l = bin < nb ? level_of_bin(bin) : 0, lj = bin < nb ? split_of(bin, l) : 0;
        const int nk = bin < nb && lj > 0 ? 1 << lj : 0, one = bin < nb && lj == 0 ? 1 : 0;
        int tn, to;
        const int fn = run_split + block_excl_scan(nk, wtot, wave, lane, tn);
        __syncthreads();  // wtot is free
        const int fo = run_other + block_excl_scan(one, wtot, wave, lane, to);
        if (bin < nb) {
            SortItem it;
            it.bh = bh;
            it.shift = lv.shift[l];
            const int off = (bin - lv.base[l]) << it.shift;
            it.t0 = lv.start[l] + off;
            it.tokens = min(1 << it.shift, lv.n[l] - off);
            it.first = bst[bin];
            it.end = bst[bin + 1];
            it.j = lj;
            for (int k = 0; k < (lj > 0 ? 1 << lj : 1); ++k) {
                it.k = k;
                list[lj > 0 ? fn + k : fo] = sort_item_pack(it);
            }
        }
        run_split += tn;
        run_other += to;
        __syncthreads();  // wtot is free for the next bins
    }
}

// The scan and the location and weight gradients (which do not depend on it) in one launch: workgroups [0, B * H) run
// the scan, the rest loc_attn_backward_kernel's grid; the scan's B * H workgroups alone would leave the GPU idle.
template <typename T, int V, int NB>
__global__ __launch_bounds__(256) void scan_loc_attn_kernel(SortParams sp, LocAttnParams lp) {
    constexpr size_t kL = kScanLds > kLocAttnLds ? kScanLds : kLocAttnLds;
    __shared__ __align__(16) unsigned char lds[kL];
    const int BH = sp.g.B * sp.g.H, wg = static_cast<int>(blockIdx.x);
    if (wg < BH)
        sort_scan_body(sp, wg, lds);
    else
        loc_attn_backward_body<T, V, NB>(lp, wg - BH, lds);
}

template <typename T>
__global__ __launch_bounds__(256) void sort_fill_kernel(SortParams sp) {
    extern __shared__ int lc[];  // [nb]: this tile's running rank per bin
    __shared__ SortLevels lv;
    const int bh = blockIdx.x / sp.qtiles, qt = blockIdx.x - bh * sp.qtiles;
    for (int i = threadIdx.x; i < sp.nb; i += 256) lc[i] = 0;
    int tk[4], lev, row;
    float cf[4];
    const bool has = sort_sample<T>(sp, bh, qt, threadIdx.x, tk, cf, lev, row);  // its loads overlap the table's
    if (threadIdx.x < kWave) sort_levels(sp, lv);
    __syncthreads();  // the level table and the cleared counters
    if (has) {
        const int* off = sp.hist + static_cast<int64_t>(bh) * sp.nb * sp.qtiles + qt;
        uint2* ent = sp.entries + static_cast<int64_t>(bh) * sp.cap;
        int bin[4], pos[4], o[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) bin[k] = tk[k] >= 0 ? sort_bin_of(lv, lev, tk[k], pos[k]) : -1;
        // the four tile starts at once (bin 0's for a dropped corner: no branch around the loads, which would each
        // be waited for at the branch's end)
#pragma unroll
        for (int k = 0; k < 4; ++k) o[k] = off[static_cast<int64_t>(bin[k] >= 0 ? bin[k] : 0) * sp.qtiles];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (bin[k] < 0) continue;
            const int rank = atomicAdd(&lc[bin[k]], 1);
            ent[o[k] + rank] =
                make_uint2(__float_as_uint(cf[k]), static_cast<unsigned>(row) << 7 | static_cast<unsigned>(pos[k]));
        }
    }
}

// Persistent: workgroup w of G (the GPU's resident count) takes items w, w + G, ... of the list (the split bins'
// items, the longest, first in each (b, h)'s part); each item's width x D float sums in LDS. A grad_out row is loaded
// by LPR = D / 4 lanes, 4 elements (8 bytes) each; the NG = 256 / LPR lane groups each own the item's tokens r with
// r % NG == grp (tokens of a neighbourhood go to different groups). Rounds of kSortChunk of the bin's entries, loaded
// 2 a thread: those in the range ranked (integer LDS atomics) by the key (r % NG) * tpg + r / NG and written to LDS in
// key order, so that each group's entries lie together, token by token; then each group streams through its own
// entries, 8 grad_out rows in flight per lane (at most 80 VGPRs and 24 KB of LDS: six workgroups a CU), adding
// each product into its tokens' LDS sums (no other group writes them, so plain LDS read-modify-writes). The sums are
// written once, in the element type. The next item is read an item ahead, and the next round's entries (of this item
// or the next) during this round, so that the loads a workgroup waits on are the grad_out rows alone. (Sums in
// registers instead, each lane holding its TB / NG tokens' 4 columns and adding every product under a per-token
// select, measured slower: 65 against 50 us at DINO B4.)
template <typename T, int D>
__global__ __launch_bounds__(256) void sort_reduce_kernel(SortParams sp) {
    constexpr int NTH = 256, VL = 4, LPR = D / VL, NG = NTH / LPR, TB = sort_bin_tokens(D), U = 8;
    constexpr int PER = kSortChunk / NTH;
    constexpr int PITCH = D + 4;  // LDS floats per token's sums: the groups' rows start in different banks
    using IO = VecIO<T, VL>;
    static_assert(D >= 8 && TB <= 128 && NG <= TB, "reduce shape");
    const Geom& g = sp.g;
    const int HD = g.H * D;
    const int tid = threadIdx.x, q = tid & (LPR - 1), grp = tid / LPR, wave = tid >> 6, lane = tid & (kWave - 1);
    const int total = sp.counters[0];
    int gi = static_cast<int>(blockIdx.x);
    if (gi >= total) return;  // uniform: before any barrier
    __shared__ __attribute__((aligned(16))) float accl[TB * PITCH];
    __shared__ uint2 sorted[kSortChunk];
    __shared__ int cnt[TB], base[TB], wtot[2];
    for (int i = tid; i < TB * PITCH / 4; i += NTH) reinterpret_cast<f32x4*>(accl)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    // a round's entries, PER a thread at clamped indexes (no branch: all in flight); n >= 1
    auto load_round = [&](uint2 (&e)[PER], int bh, int r0, int n) {
        const uint2* __restrict__ src = sp.entries + static_cast<int64_t>(bh) * sp.cap + r0;
#pragma unroll
        for (int u = 0; u < PER; ++u) e[u] = src[min(tid + u * NTH, n - 1)];
    };
    SortItem it = sort_item_unpack(sp.items[gi]);
    uint2 ex[PER];
    if (it.first < it.end) load_round(ex, it.bh, it.first, min(it.end - it.first, kSortChunk));
    while (true) {  // uniform: one item per pass
        const int gn = gi + static_cast<int>(gridDim.x);
        const SortItem itn = sort_item_unpack(sp.items[min(gn, total - 1)]);  // the next item (clamped: no branch)
        const int width = (1 << it.shift) >> it.j, lo = it.k * width;
        const int tpg = width >= NG ? width / NG : 1;  // keys per group (width and NG are powers of two)
        const T* __restrict__ go = static_cast<const T*>(sp.grad_out) + q * VL;
        bool next_loaded = false;
        for (int r0 = it.first; r0 < it.end; r0 += kSortChunk) {  // uniform: every barrier is reached by all
            const int n = min(it.end - r0, kSortChunk);
            if (tid < TB) cnt[tid] = 0;
            __syncthreads();  // the counts are clear (and the sums, after the previous item's write)
            int rk[PER], key[PER];
            bool in[PER];
#pragma unroll
            for (int u = 0; u < PER; ++u) {
                const int r = static_cast<int>(ex[u].y & 0x7fu) - lo;
                in[u] = tid + u * NTH < n && static_cast<unsigned>(r) < static_cast<unsigned>(width);
                key[u] = in[u] ? (r & (NG - 1)) * tpg + r / NG : 0;
                if (in[u]) rk[u] = atomicAdd(&cnt[key[u]], 1);
            }
            // the next round's entries: this item's, else the next item's first (else a reload of this round's)
            uint2 exn[PER];
            {
                int nbh = it.bh, nr0 = r0, nn = 1;
                if (r0 + kSortChunk < it.end) {
                    nr0 = r0 + kSortChunk;
                    nn = min(it.end - nr0, kSortChunk);
                } else if (gn < total && itn.first < itn.end) {
                    nbh = itn.bh;
                    nr0 = itn.first;
                    nn = min(itn.end - itn.first, kSortChunk);
                    next_loaded = true;
                }
                load_round(exn, nbh, nr0, nn);
            }
            __syncthreads();  // the counts are final
            if (tid < 128) {  // the first two wavefronts, every lane active: scan of the TB counts
                const int cv = tid < TB ? cnt[tid] : 0;
                const int incl = wave_incl_scan(cv);
                if (lane == kWave - 1) wtot[wave] = incl;
                if (tid < TB) base[tid] = incl - cv;
            }
            __syncthreads();
            if (tid >= kWave && tid < TB) base[tid] += wtot[0];
            __syncthreads();  // every key's start is known
#pragma unroll
            for (int u = 0; u < PER; ++u)
                if (in[u]) sorted[base[key[u]] + rk[u]] = ex[u];
            __syncthreads();  // the range's entries are in key order
            const int k0 = grp * tpg, sb = base[k0], se = base[k0 + tpg - 1] + cnt[k0 + tpg - 1];
            for (int i0 = sb; i0 < se; i0 += U) {  // this group's entries, U at a time
                typename IO::raw_t raw[U];
                float cf[U];
                int tl[U];
#pragma unroll
                for (int u = 0; u < U; ++u) {  // clamped: no branch around the loads
                    const uint2 x = sorted[min(i0 + u, se - 1)];
                    cf[u] = __uint_as_float(x.x);
                    tl[u] = static_cast<int>(x.y & 0x7fu) - lo;
                    raw[u] = IO::load(go + static_cast<int64_t>(x.y >> 7) * D);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    if (i0 + u >= se) continue;  // (no break: the loop stays unrolled, its arrays in registers)
                    float v[VL];
                    IO::unpack(raw[u], v);
                    f32x4* a = reinterpret_cast<f32x4*>(accl + tl[u] * PITCH + q * VL);
                    f32x4 s4 = *a;
#pragma unroll
                    for (int e = 0; e < VL; ++e) s4[e] += cf[u] * v[e];
                    *a = s4;
                }
            }
            __syncthreads();  // the sums are final for this round; the entries, counts and starts are free
#pragma unroll
            for (int u = 0; u < PER; ++u) ex[u] = exn[u];
        }
        // this item's rows, in the element type; each thread clears the sums it wrote out (the next item's first
        // barrier orders that before any new sums, and each thread writes out the same places in every item)
        const int b = it.bh / g.H, h = it.bh - b * g.H;
        T* __restrict__ out = static_cast<T*>(sp.grad_value) + static_cast<int64_t>(b) * g.N * HD + h * D;
        for (int i = tid; i < width * LPR; i += NTH) {
            const int tl = i / LPR, qq = i & (LPR - 1);
            f32x4* a = reinterpret_cast<f32x4*>(accl + tl * PITCH) + qq;
            const f32x4 s4 = *a;
            *a = f32x4{0.f, 0.f, 0.f, 0.f};
            if (lo + tl >= it.tokens) continue;
            const float v[VL] = {s4[0], s4[1], s4[2], s4[3]};
            IO::store(out + static_cast<int64_t>(it.t0 + lo + tl) * HD + qq * VL, v);
        }
        if (gn >= total) break;
        gi = gn;
        it = itn;
        if (!next_loaded && it.first < it.end)  // uniform: no round of the last item loaded this one's entries
            load_round(ex, it.bh, it.first, min(it.end - it.first, kSortChunk));
    }
}

// resident workgroups of 256 threads of the kernel on the current device (at least the CU count)
template <typename K>
int resident_workgroups(K kernel) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, 256, 0) != hipSuccess || per_cu < 1) per_cu = 1;
    return per_cu * cu_count();
}

template <typename T, typename A>
__global__ __launch_bounds__(256) void convert_kernel(const A* __restrict__ src, T* __restrict__ dst, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = static_cast<T>(src[i]);
}

// float32 -> 16-bit, 8 elements per thread: two 16-byte loads, one 16-byte store (n8 groups of 8; 16-byte aligned)
template <typename T>
struct Pack8 {
    T v[8];
};
template <typename T>
__global__ __launch_bounds__(256) void convert8_kernel(const f32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                       int64_t n8) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const f32x4 a = src[2 * i], b = src[2 * i + 1];
        Pack8<T> o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            o.v[e] = static_cast<T>(a[e]);
            o.v[4 + e] = static_cast<T>(b[e]);
        }
        dst[i] = __builtin_bit_cast(u32x4, o);
    }
}

// dst[c, r] = src[r, c] for a [R, Cc] matrix, through 32 x 32 LDS tiles.
template <typename T>
__global__ __launch_bounds__(256) void transpose_kernel(const T* __restrict__ src, T* __restrict__ dst, int R, int Cc) {
    __shared__ T tile[32][33];
    const int r0 = blockIdx.y * 32, c0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
    for (int i = ty; i < 32; i += 8) {
        const int r = r0 + i, c = c0 + tx;
        if (r < R && c < Cc) tile[i][tx] = src[static_cast<int64_t>(r) * Cc + c];
    }
    __syncthreads();
    for (int i = ty; i < 32; i += 8) {
        const int c = c0 + i, r = r0 + tx;
        if (r < R && c < Cc) dst[static_cast<int64_t>(c) * R + r] = tile[tx][i];
    }
}

// Weight and bias gradients, split over the M tokens: workgroup (n tile, c tile, split s) accumulates
//   part[s, n, c]  = sum over its tokens m of G[m, n] X[m, c]      (128 x 128 tile, MFMA, float32)
//   bpart[s, n]    = sum over its tokens m of G[m, n]               (c tile 0 only)
// G [M, NO] and X [M, K] are token-major, so each K-chunk of tokens is staged in LDS transposed ([n][m], [c][m]):
// MFMA fragments then hold consecutive tokens. The partials are summed in a fixed order by wgrad_reduce_kernel, so
// the result does not depend on scheduling.
struct WgradParams {
    const void* G;
    const void* X;
    float* part;
    float* bpart;
    int M, NO, K;
    int nt, ct, splits, chunk;  // tile counts, splits, tokens per split (a multiple of the MFMA K)
};

// Workgroup tile 128 (n) x 128 (c): 2 x 2 wavefronts of 64 x 64 (4 x 4 MFMA tiles), 16 MFMAs per wavefront per
// token step. Each thread stages two E-element pieces of each operand per step (KB tokens x 128 columns), from two
// consecutive tokens at the same columns: with VEC (row lengths a multiple of E, 16-byte aligned rows) as 16-byte
// loads. The pair is written transposed as E stores of two elements each ([column][token, token + 1]). The next
// step's pieces are loaded into registers while this step's MFMAs run.
constexpr int kWgTile = 128;

// two consecutive elements, stored with one 4-byte (16-bit types) or 8-byte (float32) LDS write
template <typename T>
struct alignas(2 * sizeof(T)) Pair {
    T v[2];
};

// LDS of one wgrad tile: the staged G and X slices, kWgTile rows of KBlock<T>::kK + 16 / sizeof(T) elements each
template <typename T>
constexpr size_t wgrad_slice_bytes() {
    return sizeof(T) * kWgTile * (KBlock<T>::kK + 16 / sizeof(T));
}

// Workgroup `bid` of the weight gradient's grid (tile and split), with gs and xs its two LDS slices. TW = 2 widens
// the tile to 128 (n) x 256 (c), wavefronts of 64 x 128 (32 MFMAs per token step): three quarters of the staged
// bytes, LDS reads and barriers per MFMA of the 128 x 128 tile. xs then holds 256 rows.
template <typename T, bool VEC, int TW = 1>
__device__ __forceinline__ void wgrad_tile(const WgradParams& p, int bid, T* __restrict__ gs, T* __restrict__ xs) {
    constexpr int E = 16 / static_cast<int>(sizeof(T));  // elements per 16 bytes
    constexpr int KB = KBlock<T>::kK;                     // tokens per MFMA step
    constexpr int LD = KB + E;                            // LDS pitch (elements) of a staged transposed row
    constexpr int TL = kWgTile, TC = TW * kWgTile, PIECES = KB * (TL / E) / 256;
    static_assert(PIECES == 2, "two pieces per thread");
    const int tiles = p.nt * p.ct;
    const int s = bid / tiles, tile = bid - s * tiles;
    const int n0 = (tile / p.ct) * TL, c0 = (tile % p.ct) * TC;
    const int m_begin = s * p.chunk, m_end = min(p.M, m_begin + p.chunk);
    const T* __restrict__ G = static_cast<const T*>(p.G);
    const T* __restrict__ X = static_cast<const T*>(p.X);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r16 = lane & 15, kg = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    // this thread's pieces: token rows mm[0] = 2 rp and mm[1] = 2 rp + 1, columns cc[u] = cb .. cb + E - 1; the KB / 2
    // token pairs run across consecutive lanes, so that a transposed store instruction (rows cb + e, 2 rp) spreads
    // over the LDS banks (2-way at most), where 16 column groups of one pair would meet in one or two banks
    // (X's TW column blocks of 128 are staged by the same threads, block w at columns cb + 128 w)
    const int rp = tid % (KB / 2), cb = (tid / (KB / 2)) * E;
    const int mm[PIECES] = {2 * rp, 2 * rp + 1};
    const int cc[PIECES] = {cb, cb};
    f32x4 acc[4][4 * TW];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4 * TW; ++t) acc[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float bsum = 0.f;  // thread tid < 128: column n0 + tid of G (c tile 0)
    const bool do_b = c0 == 0;

    T pg[PIECES][E], px[TW][PIECES][E];
    auto load = [&](int m0) {
#pragma unroll
        for (int u = 0; u < PIECES; ++u) {
            const int m = m0 + mm[u];
            if constexpr (VEC) {
                const u32x4 zero = {0u, 0u, 0u, 0u};
                const u32x4 vg = (m < m_end && n0 + cc[u] < p.NO)
                                     ? *reinterpret_cast<const u32x4*>(G + static_cast<int64_t>(m) * p.NO + n0 + cc[u])
                                     : zero;
                const T* eg = reinterpret_cast<const T*>(&vg);
#pragma unroll
                for (int e = 0; e < E; ++e) pg[u][e] = eg[e];
#pragma unroll
                for (int w = 0; w < TW; ++w) {
                    const int c = c0 + w * kWgTile + cc[u];
                    const u32x4 vx =
                        (m < m_end && c < p.K) ? *reinterpret_cast<const u32x4*>(X + static_cast<int64_t>(m) * p.K + c)
                                               : zero;
                    const T* ex = reinterpret_cast<const T*>(&vx);
#pragma unroll
                    for (int e = 0; e < E; ++e) px[w][u][e] = ex[e];
                }
            } else {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    const int n = n0 + cc[u] + e;
                    pg[u][e] = (m < m_end && n < p.NO) ? G[static_cast<int64_t>(m) * p.NO + n] : T(0);
#pragma unroll
                    for (int w = 0; w < TW; ++w) {
                        const int c = c0 + w * kWgTile + cc[u] + e;
                        px[w][u][e] = (m < m_end && c < p.K) ? X[static_cast<int64_t>(m) * p.K + c] : T(0);
                    }
                }
            }
        }
    };
    load(m_begin);
    for (int m0 = m_begin; m0 < m_end; m0 += KB) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            Pair<T> g2;
            g2.v[0] = pg[0][e];
            g2.v[1] = pg[1][e];
            *reinterpret_cast<Pair<T>*>(gs + (cb + e) * LD + 2 * rp) = g2;
#pragma unroll
            for (int w = 0; w < TW; ++w) {
                Pair<T> x2;
                x2.v[0] = px[w][0][e];
                x2.v[1] = px[w][1][e];
                *reinterpret_cast<Pair<T>*>(xs + (w * kWgTile + cb + e) * LD + 2 * rp) = x2;
            }
        }
        __syncthreads();
        if (m0 + KB < m_end) load(m0 + KB);  // in flight during this step's MFMAs
        if (do_b && tid < TL) {
            for (int k = 0; k < KB; ++k) bsum += static_cast<float>(gs[tid * LD + k]);
        }
        u32x4 fa[4], fb[4 * TW];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            fa[i] = *reinterpret_cast<const u32x4*>(gs + (wm * 64 + i * 16 + r16) * LD + kg * E);
#pragma unroll
        for (int t = 0; t < 4 * TW; ++t)
            fb[t] = *reinterpret_cast<const u32x4*>(xs + (wn * 64 * TW + t * 16 + r16) * LD + kg * E);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int t = 0; t < 4 * TW; ++t) acc[i][t] = KBlock<T>::mma(fa[i], fb[t], acc[i][t]);
        __syncthreads();
    }
    // acc[i][t][e]: row n0 + wm*64 + i*16 + kg*4 + e, column c0 + wn*64*TW + t*16 + r16
    float* part = p.part + static_cast<int64_t>(s) * p.NO * p.K;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4 * TW; ++t) {
            const int c = c0 + wn * 64 * TW + t * 16 + r16;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int n = n0 + wm * 64 + i * 16 + kg * 4 + e;
                if (n < p.NO && c < p.K) part[static_cast<int64_t>(n) * p.K + c] = acc[i][t][e];
            }
        }
    if (do_b && tid < TL && n0 + tid < p.NO) p.bpart[static_cast<int64_t>(s) * p.NO + n0 + tid] = bsum;
}

// Workgroups go to the XCDs round-robin (blockIdx.x % kXcds); the grid is kXcds * per_xcd workgroups, and XCD x takes
// the contiguous range [x * per_xcd, (x + 1) * per_xcd) of the (split, tile) order, so that the tiles of one split,
// which read the same token rows, share one XCD's L2 instead of pulling the rows into several.
template <typename T, bool VEC, int TW = 1>
__global__ __launch_bounds__(256) void wgrad_kernel(WgradParams p, int per_xcd) {
    __shared__ __align__(16) unsigned char lds[(1 + TW) * wgrad_slice_bytes<T>()];
    const int idx = static_cast<int>(blockIdx.x % kXcds) * per_xcd + static_cast<int>(blockIdx.x / kXcds);
    if (idx >= p.nt * p.ct * p.splits) return;  // the last XCD's spare workgroups
    wgrad_tile<T, VEC, TW>(p, idx, reinterpret_cast<T*>(lds), reinterpret_cast<T*>(lds + wgrad_slice_bytes<T>()));
}

// The input gradient's GEMM (grad_memory = G . W, on the 64 x 64 two-stage tiles the value projection's size rule
// picks below about 14000 tokens of 256 channels) and the weight gradient in one launch: they read the same G and
// nothing of each other, and each alone leaves most of the GPU idle at those sizes (about 500 and 260 workgroups of
// a few rounds of loads each). Workgroups [0, gemm_blocks) take GEMM tiles (numbered as the GEMM's own launch numbers
// them), the rest the weight gradient's tiles and splits; both run in the same 256 threads on one LDS buffer.
// WT (16-bit): the GEMM reads W as stored, [HD, C], through LDS transpose reads, instead of a transposed copy.
template <typename T, bool WT>
using InGradGemm = GemmMfmaTile<T, 4, 1, 1, 4, 4, 2, false, false, WT>;
template <typename T, bool VEC, bool WT = false>
__global__ __launch_bounds__(256) void input_weight_grad_kernel(GemmParams gp, WgradParams wp, int gemm_blocks) {
    using G = InGradGemm<T, WT>;
    constexpr size_t kW = wgrad_slice_bytes<T>();
    constexpr size_t kL = G::kLds > 2 * kW ? G::kLds : 2 * kW;
    static_assert(G::NTH == 256, "the GEMM tile runs in the weight gradient's 256 threads");
    __shared__ __align__(16) unsigned char lds[kL];
    const int b = blockIdx.x;
    if (b < gemm_blocks) {
        const int tile = tile_of(gp, b);
        if (tile >= 0) G::run(gp, tile, lds);
    } else {
        wgrad_tile<T, VEC>(wp, b - gemm_blocks, reinterpret_cast<T*>(lds), reinterpret_cast<T*>(lds + kW));
    }
}

// float64: the same sums on the vector ALUs, one thread per output of the tile
template <typename T>
__global__ __launch_bounds__(256) void wgrad_generic_kernel(WgradParams p, double* part, double* bpart) {
    const int tiles = p.nt * p.ct;
    const int s = blockIdx.x / tiles, tile = blockIdx.x - s * tiles;
    const int n0 = (tile / p.ct) * kWgTile, c0 = (tile % p.ct) * kWgTile;
    const int m_begin = s * p.chunk, m_end = min(p.M, m_begin + p.chunk);
    const T* __restrict__ G = static_cast<const T*>(p.G);
    const T* __restrict__ X = static_cast<const T*>(p.X);
    for (int o = threadIdx.x; o < kWgTile * kWgTile; o += 256) {
        const int n = n0 + o / kWgTile, c = c0 + o % kWgTile;
        if (n >= p.NO || c >= p.K) continue;
        double acc = 0, bs = 0;
        for (int m = m_begin; m < m_end; ++m) {
            const double gv = static_cast<double>(G[static_cast<int64_t>(m) * p.NO + n]);
            acc += gv * static_cast<double>(X[static_cast<int64_t>(m) * p.K + c]);
            bs += gv;
        }
        part[(static_cast<int64_t>(s) * p.NO + n) * p.K + c] = acc;
        if (c == 0) bpart[static_cast<int64_t>(s) * p.NO + n] = bs;
    }
}

// grad_W[i] = sum over splits s of part[s, i], grad_b likewise: a workgroup takes 64 outputs, its four wavefronts
// every fourth split each (reads of 64 consecutive outputs per split), and the four partial sums meet in LDS in a
// fixed order, so the result does not depend on scheduling.
template <typename T, typename P>
__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const P* __restrict__ part, const P* __restrict__ bpart,
                                                           int splits, int NO, int K, T* __restrict__ gw,
                                                           T* __restrict__ gb) {
    __shared__ P red[4][64];
    const int64_t n_out = static_cast<int64_t>(NO) * K;
    const int il = static_cast<int>(threadIdx.x) & 63, sg = static_cast<int>(threadIdx.x) >> 6;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 64 + il;
    const bool bias_block = gb != nullptr && blockIdx.x * 64 < static_cast<unsigned>(NO);
    for (int pass = 0; pass < (bias_block ? 2 : 1); ++pass) {
        const P* src = pass == 0 ? part : bpart;
        const int64_t n = pass == 0 ? n_out : NO;
        P acc = 0;
        if (i < n) {
            int s = sg;
            for (; s + 12 < splits; s += 16) {
                const P a0 = src[s * n + i], a1 = src[(s + 4) * n + i], a2 = src[(s + 8) * n + i],
                        a3 = src[(s + 12) * n + i];
                acc += a0;
                acc += a1;
                acc += a2;
                acc += a3;
            }
            for (; s < splits; s += 4) acc += src[s * n + i];
        }
        red[sg][il] = acc;
        __syncthreads();
        if (sg == 0 && i < n) {
            const P t = (red[0][il] + red[1][il]) + (red[2][il] + red[3][il]);
            if (pass == 0)
                gw[i] = static_cast<T>(t);
            else
                gb[i] = static_cast<T>(t);
        }
        __syncthreads();
    }
}

int launched(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(-3, "%s launch failed: %s", what, hipGetErrorString(e));
}

template <typename T, int CE>
int sample_backward_go(BackParams p, hipStream_t stream) {
    int lg = 1;
    while (lg * CE < p.g.D && lg < kWave) lg <<= 1;
    p.LG = lg;
    const int64_t rows = static_cast<int64_t>(p.g.B) * p.g.Q * p.g.H;
    if (rows == 0) return 0;
    hipLaunchKernelGGL((sample_backward_kernel<T, CE>), dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0,
                       stream, p);
    return launched("sample backward");
}

// one channel per lane up to D = 64 (LG = D rounded up to a power of two, the batched form), then D / 64 per lane
template <typename T>
int sample_backward_batched_go(BackParams p, hipStream_t stream) {
    int lg = 1;
    while (lg < p.g.D) lg <<= 1;
    p.LG = lg;
    const int64_t rows = static_cast<int64_t>(p.g.B) * p.g.Q * p.g.H;
    if (rows == 0) return 0;
    hipLaunchKernelGGL((sample_backward_batched_kernel<T>), dim3(static_cast<unsigned>((rows + 3) / 4)),
                       dim3(256), 0, stream, p);
    return launched("sample backward");
}

template <typename T>
int sample_backward_vec_go(BackParams p, hipStream_t stream) {
    constexpr int V = 16 / static_cast<int>(sizeof(T));
    int lg = 1;
    while (lg < p.g.D) lg <<= 1;
    p.LG = lg;
    const int64_t rows = static_cast<int64_t>(p.g.B) * p.g.Q * p.g.H;
    if (rows == 0) return 0;
    hipLaunchKernelGGL((sample_backward_vec_kernel<T, V>), dim3(static_cast<unsigned>((rows + 3) / 4)), dim3(256), 0,
                       stream, p);
    return launched("sample backward");
}

// The bucketed scatter pays where the corners of neighbouring queries overlap: at least 16 corner hits per token
// and head on average (encoder self-attention: 64 at DINO's 4 levels x 4 points; decoders: 2-4).
inline bool bucket_scatter_pays(const Geom& g) {
    return is_pow2(g.D) && g.D >= 4 && g.D <= 64 && g.P > 0 && g.N > 0 && g.LP > 0 && g.LP <= 256 &&
           static_cast<int64_t>(g.Q) * g.LP * 4 >= int64_t{16} * g.N;
}

template <typename T>
int scatter_bucket_go(const BackParams& p, hipStream_t stream) {
    const Geom& g = p.g;
    BucketParams bp{p.loc, p.attn, p.grad_out, p.grad_value, g, 0, 0, 0, 0, {}, {}};
    constexpr int NTH = 512;
    // QT rows of one (row, sample) per thread, QT * P * 4 corner entries per level, QT * D grad_out floats
    bp.QT = 32;
    if (bp.QT > NTH / g.LP) bp.QT = NTH / g.LP;
    if (bp.QT > kBucketEnt / (4 * g.P)) bp.QT = kBucketEnt / (4 * g.P);
    if (bp.QT * g.D > 2 * NTH) bp.QT = 2 * NTH / g.D;
    if (bp.QT < 1) return set_error(-1, "sample backward: no bucket shape for these sizes");
    bp.qtiles = (g.Q + bp.QT - 1) / bp.QT;
    const int64_t units = static_cast<int64_t>(g.B) * g.H * bp.qtiles;
    if (units == 0) return 0;
    if (units > (int64_t{1} << 30)) return set_error(-1, "sample backward: too many query tiles");
    bp.units = static_cast<int>(units);
    bp.per_xcd = static_cast<int>((units + kXcds - 1) / kXcds);
    bp.d_lp = make_fastdiv(static_cast<uint32_t>(g.LP));
    bp.d_p = make_fastdiv(static_cast<uint32_t>(g.P));
    // Self-attention (as many queries as tokens, 32-query tiles): 8 x 4-pixel tiles of each level's map, which touch
    // fewer pixels than 32 queries along one map row and never wrap a row; the tile count depends on the level sizes,
    // which stay on the device, so a grid of three workgroups per CU (what the kernel's registers allow) strides
    // over them
    if (g.Q == g.N && bp.QT == kTileW * kTileH && static_cast<int64_t>(g.B) * g.H * g.N <= (int64_t{1} << 30)) {
        int64_t grid = static_cast<int64_t>(g.B) * g.H * ((g.N + bp.QT - 1) / bp.QT + 2 * g.L);
        const int64_t resident = 3 * static_cast<int64_t>(cu_count());
        if (grid > resident) grid = resident;
        hipLaunchKernelGGL((scatter_bucket_kernel<T, NTH, true>), dim3(static_cast<unsigned>(grid)), dim3(NTH), 0,
                           stream, bp);
        return launched("sample backward scatter");
    }
    hipLaunchKernelGGL((scatter_bucket_kernel<T, NTH, false>), dim3(static_cast<unsigned>(bp.per_xcd * kXcds)),
                       dim3(NTH), 0, stream, bp);
    return launched("sample backward scatter");
}

// loc_attn_backward_kernel's shape: RB = 256 / LP rows a workgroup, SG corner groups a row (every thread a lane
// where RB * DV <= 256); 1 without launching when the kernel does not fit (the caller then takes
// sample_backward_vec_kernel or the atomic scatter)
// loc_attn_backward_kernel's parameters for p; 1 when the kernel does not fit (see above)
template <typename T>
int loc_attn_plan(const BackParams& p, LocAttnParams& lp) {
    constexpr int V = 16 / static_cast<int>(sizeof(T)), NTH = 256;
    const Geom& g = p.g;
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
    const int64_t vbytes = static_cast<int64_t>(g.B) * g.N * g.H * g.D * static_cast<int64_t>(sizeof(T));
    const int DV = g.D / V;
    // 16-byte value and grad_out loads: D a multiple of V (DV a power of two), 16-byte aligned rows
    if (g.D % V != 0 || !is_pow2(DV) || DV > 16 || reinterpret_cast<uintptr_t>(p.value) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(p.grad_out) % 16 != 0 || g.LP <= 0 || g.LP > NTH ||
        rows * g.LP >= (int64_t{1} << 31) || vbytes >= (int64_t{1} << 31))
        return 1;
    lp = LocAttnParams{p, 0, 0, 0, 0, 0, {}, {}, {}, {}, {}};
    lp.RB = NTH / g.LP;
    lp.SG = NTH / (lp.RB * DV) > 0 ? NTH / (lp.RB * DV) : 1;
    const int64_t blocks = (rows + lp.RB - 1) / lp.RB;
    lp.blocks = static_cast<int>(blocks);
    lp.per_xcd = static_cast<int>((blocks + kXcds - 1) / kXcds);
    lp.val_bytes = static_cast<int>(vbytes);
    lp.d_lp = make_fastdiv(static_cast<uint32_t>(g.LP));
    lp.d_gs = make_fastdiv(static_cast<uint32_t>(DV * lp.SG));
    lp.d_dv = make_fastdiv(static_cast<uint32_t>(DV));
    lp.d_q = make_fastdiv(static_cast<uint32_t>(g.Q));
    lp.d_h = make_fastdiv(static_cast<uint32_t>(g.H));
    return 0;
}

template <typename T>
int loc_attn_backward_go(const BackParams& p, hipStream_t stream) {
    constexpr int V = 16 / static_cast<int>(sizeof(T));
    LocAttnParams lp;
    const int rc = loc_attn_plan<T>(p, lp);
    if (rc != 0) return rc;
    if (lp.blocks == 0) return 0;
    hipLaunchKernelGGL((loc_attn_backward_kernel<T, V, 8>), dim3(static_cast<unsigned>(lp.per_xcd * kXcds)), dim3(256),
                       0, stream, lp);
    return launched("sample backward locations");
}

// The binned path (sort_count_kernel ... sort_reduce_kernel) for 16-bit types at decoder densities, with the location
// and weight gradients from loc_attn_backward_kernel; grad_value (the element type, 8-byte aligned) is written
// directly. Returns 1 without launching when it does not apply: too few corners to pay for its five launches, a dense
// problem (the bucketed scatter's), a head width other than 8..64 (a power of two), more than kSortMaxBins bins or
// 2^25 rows, scratch that does not fit in the accumulator buffer (acc_bytes), or shapes loc_attn_backward_kernel
// does not take (value or grad_out rows not 16-byte aligned).
constexpr int64_t kSortMinCorners = int64_t{1} << 18;

template <typename T>
int sample_backward_sorted(const BackParams& p, void* grad_value_t, int64_t acc_bytes, hipStream_t stream) {
    const Geom& g = p.g;
    if (grad_value_t == nullptr || grad_value_t == p.grad_value || reinterpret_cast<uintptr_t>(grad_value_t) % 8 != 0 ||
        reinterpret_cast<uintptr_t>(p.grad_value) % 16 != 0 || !is_pow2(g.D) || g.D < 8 || g.D > 64 || g.LP <= 0 ||
        g.LP > 256 || g.L > kMaxLevelPoints || bucket_scatter_pays(g))
        return 1;
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q * g.H;
    if (rows * g.LP * 4 < kSortMinCorners || rows >= (int64_t{1} << 25)) return 1;
    SortParams sp{};
    sp.loc = p.loc;
    sp.attn = p.attn;
    sp.grad_out = p.grad_out;
    sp.grad_value = grad_value_t;
    sp.g = g;
    sp.QT = 256 / g.LP;
    sp.qtiles = (g.Q + sp.QT - 1) / sp.QT;
    sp.tb_shift = ilog2(sort_bin_tokens(g.D));
    sp.cap = static_cast<int64_t>(g.Q) * g.LP * 4;
    const int64_t BH = static_cast<int64_t>(g.B) * g.H;
    if (sp.cap >= (int64_t{1} << 31) || BH >= (int64_t{1} << 23)) return 1;
    // the narrowest bins (8 tokens or more) for which the bins (N / 2^min_shift + L at most: each level's last bin
    // may be partial) stay within kSortMaxBins and the scratch (entries, items, counts, starts) fits in acc_bytes;
    // items: one per bin, or 2^j < 2 count / kSortChunk for a split bin, so at most nb + 2 cap / kSortChunk
    const int64_t ent_bytes = (BH * sp.cap * 8 + 15) / 16 * 16;
    int64_t nb = 0, maxch = 0, item_bytes = 0;
    for (sp.min_shift = 3;; ++sp.min_shift) {
        if (sp.min_shift > sp.tb_shift) return 1;
        nb = ((static_cast<int64_t>(g.N) >> sp.min_shift) + 1) + g.L;
        maxch = nb + 2 * sp.cap / kSortChunk + 1;
        item_bytes = BH * maxch * 16;
        const int64_t ints = BH * nb * sp.qtiles + BH * (nb + 1) + 1;
        if (nb <= kSortMaxBins && nb * sp.qtiles < (int64_t{1} << 30) && BH * maxch < (int64_t{1} << 31) &&
            ent_bytes + item_bytes + 4 * ints <= acc_bytes)
            break;
    }
    sp.nb = static_cast<int>(nb);
    sp.maxch = static_cast<int>(maxch);
    // the location and weight gradients' plan (1: its 16-byte loads do not fit these sizes); they run beside the scan
    LocAttnParams lp;
    const int rc = loc_attn_plan<T>(p, lp);
    if (rc != 0) return rc;
    unsigned char* scratch = static_cast<unsigned char*>(p.grad_value);  // 16-byte aligned (checked above)
    sp.entries = reinterpret_cast<uint2*>(scratch);
    sp.items = reinterpret_cast<uint4*>(scratch + ent_bytes);
    sp.hist = reinterpret_cast<int*>(scratch + ent_bytes + item_bytes);
    sp.bin_start = sp.hist + BH * nb * sp.qtiles;
    sp.counters = sp.bin_start + BH * (nb + 1);
    sp.d_lp = make_fastdiv(static_cast<uint32_t>(g.LP));
    const unsigned tiles = static_cast<unsigned>(BH * sp.qtiles);
    const size_t lds = static_cast<size_t>(nb) * sizeof(int);
    hipLaunchKernelGGL(sort_count_kernel<T>, dim3(tiles), dim3(256), lds, stream, sp);
    int r2 = launched("sample backward count");
    if (r2 != 0) return r2;
    {  // the scan and the location and weight gradients in one launch
        constexpr int V = 16 / static_cast<int>(sizeof(T));
        const unsigned lblocks = lp.blocks > 0 ? static_cast<unsigned>(lp.per_xcd * kXcds) : 0u;
        hipLaunchKernelGGL((scan_loc_attn_kernel<T, V, 8>), dim3(static_cast<unsigned>(BH) + lblocks), dim3(256), 0,
                           stream, sp, lp);
    }
    r2 = launched("sample backward scan and locations");
    if (r2 != 0) return r2;
    hipLaunchKernelGGL(sort_fill_kernel<T>, dim3(tiles), dim3(256), lds, stream, sp);
    r2 = launched("sample backward fill");
    if (r2 != 0) return r2;
    // persistent: the resident count (at most the items' bound)
    auto go = [&](auto kernel) {
        static const int resident = resident_workgroups(kernel);
        const int64_t grid = std::min<int64_t>(resident, BH * maxch);
        hipLaunchKernelGGL(kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, stream, sp);
    };
    switch (g.D) {
        case 8: go(sort_reduce_kernel<T, 8>); break;
        case 16: go(sort_reduce_kernel<T, 16>); break;
        case 32: go(sort_reduce_kernel<T, 32>); break;
        default: go(sort_reduce_kernel<T, 64>); break;
    }
    return launched("sample backward reduce");
}

template <typename T>
int sample_backward_t(const BackParams& p, hipStream_t stream) {
    constexpr int V = 16 / static_cast<int>(sizeof(T));
    if constexpr (sizeof(T) <= 4) {
        // 16-byte value loads need D a multiple of V and 16-byte aligned value rows
        if (p.g.D <= 64 && p.g.D % V == 0 && is_pow2(p.g.D / V) && reinterpret_cast<uintptr_t>(p.value) % 16 == 0 &&
            reinterpret_cast<uintptr_t>(p.grad_out) % 16 == 0) {
            if (!bucket_scatter_pays(p.g)) return sample_backward_vec_go<T>(p, stream);
            int rc = loc_attn_backward_go<T>(p, stream);
            if (rc == 1) {
                BackParams q = p;
                q.scatter = 0;  // the dot products and the location and weight gradients only
                rc = sample_backward_vec_go<T>(q, stream);
            }
            return rc != 0 ? rc : scatter_bucket_go<T>(p, stream);
        }
    }
    if (p.g.D <= 64) return sample_backward_batched_go<T>(p, stream);
    if (p.g.D <= 128) return sample_backward_go<T, 2>(p, stream);
    return sample_backward_go<T, 4>(p, stream);
}

}  // namespace

int launch_sample_backward(int dtype, const void* value, const Geom& g, const void* loc, const void* attn,
                           const void* grad_out, void* grad_value, void* grad_value_t, void* grad_loc, void* grad_attn,
                           hipStream_t stream, bool* direct) {
    if (g.D > kWave * 4) return set_error(-1, "sample backward: head dim %d > %d", g.D, kWave * 4);
    const int acc = dtype == kF64 ? 8 : 4;
    const int64_t acc_bytes = static_cast<int64_t>(g.B) * g.N * g.H * g.D * acc;
    BackParams p{value, loc, attn, grad_out, grad_value, grad_loc, grad_attn, g, 1};
    *direct = false;
    if ((dtype == kF16 || dtype == kBF16) && (reinterpret_cast<uintptr_t>(grad_value) % 8) == 0) {
        const int rs = dtype == kF16 ? sample_backward_sorted<f16>(p, grad_value_t, acc_bytes, stream)
                                     : sample_backward_sorted<bf16>(p, grad_value_t, acc_bytes, stream);
        if (rs != 1) {
            *direct = rs == 0;
            return rs;
        }
    }
    const int rc = launch_zero(grad_value, acc_bytes, stream);
    if (rc != 0) return rc;
    switch (dtype) {
        case kF32: return sample_backward_t<float>(p, stream);
        case kF16: return sample_backward_t<f16>(p, stream);
        case kBF16: return sample_backward_t<bf16>(p, stream);
        case kF64: return sample_backward_t<double>(p, stream);
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
}

int launch_convert(int dtype, const void* src_acc, void* dst, int64_t n, hipStream_t stream) {
    if (n <= 0) return 0;
    const bool vec = (dtype == kF16 || dtype == kBF16) && n % 8 == 0 &&
                     (reinterpret_cast<uintptr_t>(src_acc) | reinterpret_cast<uintptr_t>(dst)) % 16 == 0;
    if (vec) {
        int64_t blocks = (n / 8 + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        const dim3 grid(static_cast<unsigned>(blocks));
        if (dtype == kF16)
            hipLaunchKernelGGL(convert8_kernel<f16>, grid, dim3(256), 0, stream, static_cast<const f32x4*>(src_acc),
                               static_cast<u32x4*>(dst), n / 8);
        else
            hipLaunchKernelGGL(convert8_kernel<bf16>, grid, dim3(256), 0, stream, static_cast<const f32x4*>(src_acc),
                               static_cast<u32x4*>(dst), n / 8);
        return launched("convert");
    }
    int64_t blocks = (n + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (dtype) {
        case kF32: hipLaunchKernelGGL((convert_kernel<float, float>), grid, dim3(256), 0, stream,
                                      static_cast<const float*>(src_acc), static_cast<float*>(dst), n); break;
        case kF16: hipLaunchKernelGGL((convert_kernel<f16, float>), grid, dim3(256), 0, stream,
                                      static_cast<const float*>(src_acc), static_cast<f16*>(dst), n); break;
        case kBF16: hipLaunchKernelGGL((convert_kernel<bf16, float>), grid, dim3(256), 0, stream,
                                       static_cast<const float*>(src_acc), static_cast<bf16*>(dst), n); break;
        case kF64: hipLaunchKernelGGL((convert_kernel<double, double>), grid, dim3(256), 0, stream,
                                      static_cast<const double*>(src_acc), static_cast<double*>(dst), n); break;
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
    return launched("convert");
}

int launch_transpose(int dtype, const void* src, void* dst, int64_t R, int64_t Cc, hipStream_t stream) {
    if (R * Cc == 0) return 0;
    const dim3 grid(static_cast<unsigned>((Cc + 31) / 32), static_cast<unsigned>((R + 31) / 32));
    const int r = static_cast<int>(R), c = static_cast<int>(Cc);
    switch (dtype) {
        case kF32: hipLaunchKernelGGL(transpose_kernel<float>, grid, dim3(256), 0, stream,
                                      static_cast<const float*>(src), static_cast<float*>(dst), r, c); break;
        case kF16: hipLaunchKernelGGL(transpose_kernel<f16>, grid, dim3(256), 0, stream,
                                      static_cast<const f16*>(src), static_cast<f16*>(dst), r, c); break;
        case kBF16: hipLaunchKernelGGL(transpose_kernel<bf16>, grid, dim3(256), 0, stream,
                                       static_cast<const bf16*>(src), static_cast<bf16*>(dst), r, c); break;
        case kF64: hipLaunchKernelGGL(transpose_kernel<double>, grid, dim3(256), 0, stream,
                                      static_cast<const double*>(src), static_cast<double*>(dst), r, c); break;
        default: return set_error(-2, "unknown dtype code %d", dtype);
    }
    return launched("transpose");
}

// grad_memory = G . W (through W^T, as td_input_grad computes it) and the weight gradient of the same G: where the
// value projection's size rule picks the 64 x 64 two-stage tiles for the input gradient, its tiles and the weight
// gradient's run in one launch (input_weight_grad_kernel); otherwise the two run one after the other. The workspace
// is the weight gradient's (td_weight_grad_workspace). M, HD and C are positive.
int launch_input_weight_grad(int dtype, const void* G, const void* W, void* Wt, const void* X, void* gm, void* gw,
                             void* gb, int64_t M, int64_t HD, int64_t C, void* workspace, int64_t ws_bytes,
                             hipStream_t stream) {
    if (value_proj_plan(dtype, G, Wt, nullptr, gm, M, HD, C, 0, 0) == 25) {
        // 16-bit with C a multiple of 8 and W 16-byte aligned: the GEMM reads W as stored (no transpose launch,
        // Wt is left unwritten)
        const bool stored = (dtype == kF16 || dtype == kBF16) && C % 8 == 0 &&
                            reinterpret_cast<uintptr_t>(W) % 16 == 0;
        if (!stored) {
            const int rc = launch_transpose(dtype, W, Wt, HD, C, stream);
            if (rc != 0) return rc;
        }
        const GemmParams gp{G, stored ? W : Wt, nullptr, gm, static_cast<int>(M), static_cast<int>(HD),
                            static_cast<int>(C), 0, 0, 0};
        return launch_wgrad(dtype, G, X, gw, gb, M, HD, C, workspace, ws_bytes, stream, &gp, stored);
    }
    // the streaming GEMM (16-bit, C = 256, HD = 128 or 256, many tokens) reads W as stored too
    const GemmParams sp{G, W, nullptr, gm, static_cast<int>(M), static_cast<int>(HD), static_cast<int>(C), 0, 0, 0};
    int rc = 0;
    if (value_proj_plan(dtype, G, W, nullptr, gm, M, HD, C, 0, 0) == 22 && gemm_stream_fits(dtype, sp)) {
        rc = launch_gemm_stream(dtype, sp, stream, true);
        if (rc != 0) return rc;
        return launch_wgrad(dtype, G, X, gw, gb, M, HD, C, workspace, ws_bytes, stream);
    }
    rc = launch_transpose(dtype, W, Wt, HD, C, stream);
    if (rc != 0) return rc;
    rc = launch_value_proj(dtype, G, Wt, nullptr, gm, M, HD, C, stream);
    if (rc != 0) return rc;
    return launch_wgrad(dtype, G, X, gw, gb, M, HD, C, workspace, ws_bytes, stream);
}

// Column tiles of 256 (TW = 2) for the weight gradient's own launch from this many input channels on: training
// step at C = 1024 bf16 B2 Q300 544.1 -> 494.1 us; from 256 channels on, DINO B4 Q900 168.7 -> 176.1 and RT-DETR bf16
// B8 124.6 -> 129.0 (half the tiles, so twice the splits and partials)
constexpr int64_t kWgWideMinK = 512;

int wgrad_width(int64_t K, int dtype) { return dtype != kF64 && K >= kWgWideMinK ? 2 : 1; }

// Split count of the weight gradient: about 512 workgroups (1024 for large outputs), at least four token steps per
// split (64 tokens in float32, 128 otherwise). Measured on the training step at 8400 tokens (256 x 256), against 256
// tokens per split: float32 117.0 -> 99.0 us with 64-token splits (105.8 with 128), 16-bit 63.3 -> 62.7 with 128
// (63.4 with 64); problems of 32768 tokens and more already had their 512 workgroups.
static void wgrad_split(int64_t M, int64_t NO, int64_t K, int dtype, int tw, int* splits, int* chunk) {
    const int64_t tiles = ((NO + kWgTile - 1) / kWgTile) * ((K + tw * kWgTile - 1) / (tw * kWgTile));
    const int kb = dtype == kF32 ? 16 : 32;
    // 1024 workgroups from 64 output tiles (C = 1024): training step at C = 1024 bf16 B2 Q300 913.0 -> 895.2 us; at
    // 4 tiles (C = 256) 1024 lost 1.5-5% (DINO B4 Q900, bf16 B8 Q300, the DINO encoder: more partials to reduce)
    const int64_t target = tiles >= 64 ? 1024 : 512;
    int64_t s = (target + tiles - 1) / tiles;
    // at least four token steps per split; in 16 bits below 16384 tokens (where the input gradient's GEMM shares the
    // launch) eight: training step at RT-DETR B1 fp16 Q300 55.6 -> 55.1 us, Q100 48.7 -> 48.2 (half the partials to
    // reduce); float32 lost with eight (95.2 -> 97.4)
    const int64_t min_tok = kb * ((dtype == kF16 || dtype == kBF16) && M < 16384 ? 8 : 4);
    const int64_t max_s = (M + min_tok - 1) / min_tok;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    int64_t c = (M + s - 1) / s;
    c = (c + kb - 1) / kb * kb;
    s = c > 0 ? (M + c - 1) / c : 1;
    if (s < 1) s = 1;
    *splits = static_cast<int>(s);
    *chunk = static_cast<int>(c > 0 ? c : kb);
}

// Splits, tokens per split and workspace of the weight gradient's own launch; the workspace also covers the 128-wide
// tiles of the launch combined with the input gradient's GEMM.
void wgrad_plan(int64_t M, int64_t NO, int64_t K, int dtype, int* splits, int* chunk, int64_t* ws_bytes) {
    int s1 = 1, c1 = 32;
    wgrad_split(M, NO, K, dtype, 1, &s1, &c1);
    const int tw = wgrad_width(K, dtype);
    *splits = s1;
    *chunk = c1;
    if (tw != 1) wgrad_split(M, NO, K, dtype, tw, splits, chunk);
    const int64_t elem = dtype == kF64 ? 8 : 4;
    *ws_bytes = (s1 > *splits ? s1 : *splits) * (NO * K + NO) * elem;
}

int launch_wgrad(int dtype, const void* G, const void* X, void* gw, void* gb, int64_t M, int64_t NO, int64_t K,
                 void* workspace, int64_t ws_bytes, hipStream_t stream, const GemmParams* with_gemm, bool gemm_wt) {
    int splits = 1, chunk = 32;
    int64_t need = 0;
    wgrad_plan(M, NO, K, dtype, &splits, &chunk, &need);
    if (workspace == nullptr || ws_bytes < need)
        return set_error(-4, "weight gradient: workspace of %lld bytes needed, %lld given", static_cast<long long>(need),
                         static_cast<long long>(ws_bytes));
    if (NO * K == 0) return 0;
    const int tw = with_gemm != nullptr ? 1 : wgrad_width(K, dtype);
    if (tw != wgrad_width(K, dtype)) wgrad_split(M, NO, K, dtype, tw, &splits, &chunk);
    WgradParams p{G, X, nullptr, nullptr, static_cast<int>(M), static_cast<int>(NO), static_cast<int>(K),
                  static_cast<int>((NO + kWgTile - 1) / kWgTile),
                  static_cast<int>((K + tw * kWgTile - 1) / (tw * kWgTile)), splits, chunk};
    const int64_t n_out = NO * K;
    const dim3 grid(static_cast<unsigned>(static_cast<int64_t>(p.nt) * p.ct * splits));
    const dim3 rgrid(static_cast<unsigned>((n_out + 63) / 64));
    if (dtype == kF64) {
        double* part = static_cast<double*>(workspace);
        double* bpart = part + static_cast<int64_t>(splits) * n_out;
        if (M == 0) {
            const int rc = launch_zero(gw, n_out * 8, stream);
            return rc != 0 || gb == nullptr ? rc : launch_zero(gb, NO * 8, stream);
        }
        hipLaunchKernelGGL(wgrad_generic_kernel<double>, grid, dim3(256), 0, stream, p, part, bpart);
        int rc = launched("weight gradient");
        if (rc != 0) return rc;
        hipLaunchKernelGGL((wgrad_reduce_kernel<double, double>), rgrid, dim3(256), 0, stream, part, bpart, splits,
                           p.NO, p.K, static_cast<double*>(gw), static_cast<double*>(gb));
        return launched("weight gradient reduce");
    }
    p.part = static_cast<float*>(workspace);
    p.bpart = p.part + static_cast<int64_t>(splits) * n_out;
    const int es = dtype == kF32 ? 4 : 2;
    if (M == 0) {
        const int rc = launch_zero(gw, n_out * es, stream);
        return rc != 0 || gb == nullptr ? rc : launch_zero(gb, NO * es, stream);
    }
    const int E = dtype == kF32 ? 4 : 8;
    const bool vec = NO % E == 0 && K % E == 0 &&
                     ((reinterpret_cast<uintptr_t>(G) | reinterpret_cast<uintptr_t>(X)) % 16) == 0;
    if (with_gemm != nullptr) {
        // the input gradient's GEMM tiles first, numbered as its own launch numbers them, then the weight gradient's
        GemmParams gp = *with_gemm;
        gp.mt = (gp.M + 63) / 64;
        gp.nt = (gp.NO + 63) / 64;
        gp.per_xcd = static_cast<int>((static_cast<int64_t>(gp.mt) * gp.nt + kXcds - 1) / kXcds);
        const int gemm_blocks = gp.per_xcd * kXcds;
        const dim3 cgrid(static_cast<unsigned>(gemm_blocks + static_cast<int64_t>(grid.x)));
        switch (dtype * 2 + (vec ? 1 : 0)) {
            case kF32 * 2:
                hipLaunchKernelGGL((input_weight_grad_kernel<float, false>), cgrid, dim3(256), 0, stream, gp, p,
                                   gemm_blocks);
                break;
            case kF32 * 2 + 1:
                hipLaunchKernelGGL((input_weight_grad_kernel<float, true>), cgrid, dim3(256), 0, stream, gp, p,
                                   gemm_blocks);
                break;
            case kF16 * 2:
                if (gemm_wt)
                    hipLaunchKernelGGL((input_weight_grad_kernel<f16, false, true>), cgrid, dim3(256), 0, stream, gp,
                                       p, gemm_blocks);
                else
                    hipLaunchKernelGGL((input_weight_grad_kernel<f16, false>), cgrid, dim3(256), 0, stream, gp, p,
                                       gemm_blocks);
                break;
            case kF16 * 2 + 1:
                if (gemm_wt)
                    hipLaunchKernelGGL((input_weight_grad_kernel<f16, true, true>), cgrid, dim3(256), 0, stream, gp,
                                       p, gemm_blocks);
                else
                    hipLaunchKernelGGL((input_weight_grad_kernel<f16, true>), cgrid, dim3(256), 0, stream, gp, p,
                                       gemm_blocks);
                break;
            case kBF16 * 2:
                if (gemm_wt)
                    hipLaunchKernelGGL((input_weight_grad_kernel<bf16, false, true>), cgrid, dim3(256), 0, stream, gp,
                                       p, gemm_blocks);
                else
                    hipLaunchKernelGGL((input_weight_grad_kernel<bf16, false>), cgrid, dim3(256), 0, stream, gp, p,
                                       gemm_blocks);
                break;
            case kBF16 * 2 + 1:
                if (gemm_wt)
                    hipLaunchKernelGGL((input_weight_grad_kernel<bf16, true, true>), cgrid, dim3(256), 0, stream, gp,
                                       p, gemm_blocks);
                else
                    hipLaunchKernelGGL((input_weight_grad_kernel<bf16, true>), cgrid, dim3(256), 0, stream, gp, p,
                                       gemm_blocks);
                break;
            default: return set_error(-2, "unknown dtype code %d", dtype);
        }
    } else {
        const int per_xcd = static_cast<int>((static_cast<int64_t>(grid.x) + kXcds - 1) / kXcds);
        const dim3 xgrid(static_cast<unsigned>(per_xcd * kXcds));
        switch ((dtype * 2 + (vec ? 1 : 0)) * 2 + (tw == 2 ? 1 : 0)) {
#define TD_WG(code, T, V)                                                                                          \
    case (code * 2 + V) * 2:                                                                                       \
        hipLaunchKernelGGL((wgrad_kernel<T, V, 1>), xgrid, dim3(256), 0, stream, p, per_xcd);                      \
        break;                                                                                                     \
    case (code * 2 + V) * 2 + 1:                                                                                   \
        hipLaunchKernelGGL((wgrad_kernel<T, V, 2>), xgrid, dim3(256), 0, stream, p, per_xcd);                      \
        break;
            TD_WG(kF32, float, false)
            TD_WG(kF32, float, true)
            TD_WG(kF16, f16, false)
            TD_WG(kF16, f16, true)
            TD_WG(kBF16, bf16, false)
            TD_WG(kBF16, bf16, true)
#undef TD_WG
            default: return set_error(-2, "unknown dtype code %d", dtype);
        }
    }
    int rc = launched(with_gemm != nullptr ? "input and weight gradients" : "weight gradient");
    if (rc != 0) return rc;
    switch (dtype) {
        case kF32: hipLaunchKernelGGL((wgrad_reduce_kernel<float, float>), rgrid, dim3(256), 0, stream, p.part,
                                      p.bpart, splits, p.NO, p.K, static_cast<float*>(gw), static_cast<float*>(gb));
            break;
        case kF16: hipLaunchKernelGGL((wgrad_reduce_kernel<f16, float>), rgrid, dim3(256), 0, stream, p.part, p.bpart,
                                      splits, p.NO, p.K, static_cast<f16*>(gw), static_cast<f16*>(gb));
            break;
        default: hipLaunchKernelGGL((wgrad_reduce_kernel<bf16, float>), rgrid, dim3(256), 0, stream, p.part,
                                    p.bpart, splits, p.NO, p.K, static_cast<bf16*>(gw), static_cast<bf16*>(gb));
            break;
    }
    return launched("weight gradient reduce");
}

}  // namespace td
