// Shared device code for the gfx950 kernels: element types, vector loads, the bilinear corner rule and
// wavefront (64-lane) cross-lane helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace td {

constexpr int kWave = 64;
constexpr int kXcds = 8;  // MI355X: workgroups are dealt to 8 XCDs (each with its own L2) round-robin
constexpr int kMaxLevelPoints = 64;  // L * P per head (reference csrc/ma_deform_fused.cu:27)
constexpr int kMaxChannels = 8192;   // C in fused mode (reference csrc/ma_deform_fused.cu:28)

typedef _Float16 f16;
typedef __bf16 bf16;
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef bf16 bf16x8 __attribute__((ext_vector_type(8)));

// n / d for 0 <= n < 2^31 and 1 <= d < 2^31 by a multiply-high, an add and a shift (Granlund and Montgomery,
// "Division by invariant integers using multiplication", PLDI 1994, the round-up form): with l = ceil(log2 d) and
// mul = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, mul) + n) >> l; mul < 2^32, and the sum stays below 2^32
// because mulhi(n, mul) < n < 2^31.
struct FastDiv {
    uint32_t mul = 1, shift = 0;
};
inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((uint64_t{1} << l) < d) ++l;
    FastDiv f;
    f.mul = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
    f.shift = l;
    return f;
}
__device__ __forceinline__ uint32_t fast_div(const FastDiv& f, uint32_t n) {
    return (__umulhi(n, f.mul) + n) >> f.shift;
}

// Accumulation type: float for float/half/bfloat16, double for double.
template <typename T>
struct AccOf {
    using type = float;
};
template <>
struct AccOf<double> {
    using type = double;
};

template <typename A, typename T>
__device__ __forceinline__ A cvt(T v) {
    return static_cast<A>(v);
}

// Level geometry and sizes shared by all kernels. shapes/starts are device pointers (int64), read on the
// device so that a call never reads level sizes on the host (safe under stream capture).
struct Geom {
    const int64_t* shapes;  // [L, 2] (height, width)
    const int64_t* starts;  // [L] first token of each level
    int B, Q, N, H, D, L, P;
    const uint8_t* mask = nullptr;  // [B, N] padding mask (non-zero = padded token, value zero) or null
    int LP = 0;                     // samples per row: L * P, or the sum of per-level point counts
    int discrete = 0;               // 1: nearest-pixel sampling (D-FINE's "discrete" method) instead of bilinear
    int loc_acc = 0;                // 1: locations and weights are in the accumulation type (float; double for
                                    // float64) instead of the element type (computed by the query prologue)
    int value_hm = 0;               // sampling: 1 when value is head-major [B, H, N, D] instead of [B, N, H * D]
    uint8_t level_end[kMaxLevelPoints] = {};  // per-level point counts (P == 0): first sample after level l

    // true when the general corner rule is needed (padding mask, per-level point counts, discrete sampling or
    // locations in the accumulation type)
    bool general() const { return mask != nullptr || P == 0 || discrete != 0 || loc_acc != 0; }
};

// Fills Geom::LP (and Geom::level_end with P = 0 when `points` gives per-level counts; points == nullptr keeps P
// points on every level). Returns false when the total exceeds kMaxLevelPoints.
inline bool set_levels(Geom& g, const int64_t* points) {
    if (points == nullptr) {
        g.LP = g.L * g.P;
        return g.LP <= kMaxLevelPoints;
    }
    int64_t j = 0;
    for (int l = 0; l < g.L; ++l) {
        if (points[l] < 0 || j + points[l] > kMaxLevelPoints) return false;
        j += points[l];
        g.level_end[l] = static_cast<uint8_t>(j);
    }
    g.P = 0;
    g.LP = static_cast<int>(j);
    return true;
}

// Level of sample j: j / P for P points per level; otherwise the number of levels that end at or before j
// (uniform loop over levels, so the counts are read as scalars).
__device__ __forceinline__ int level_of(const Geom& g, int j) {
    if (g.P > 0) return j / g.P;
    int l = 0;
    for (int i = 0; i + 1 < g.L; ++i) l += j >= g.level_end[i];
    return l;
}

// One gathered corner: token index (-1 when the corner lies outside its level map or outside [0, N)) and
// its weight (attention weight x bilinear weight; 0 when outside).
template <typename A>
struct Corner {
    int tok;
    A w;
};

// The four bilinear corners of one sample of row `row` = (b * Q + q) * H + h on level l, at normalised location
// (lx, ly) with attention weight w. Restates the reference's corner rule (csrc/ma_deform_fused.cu:81-100): pixel
// coordinate x = lx * W_l - 0.5 (align_corners=False), clamped to [-2, W_l + 1] before the integer conversion so
// that far-away, infinite or NaN locations sample nothing; corner k has dx = k & 1, dy = k >> 1; a corner counts
// only if it lies inside the level map and its token t = start_l + y * W_l + x lies in [0, N). With a padding mask,
// a corner on a padded token counts as outside too: its value row is zero (value.masked_fill(mask, 0) after the
// projection), so in fused mode it drops both W . memory[t] and its share of the bias.
//
// Discrete method (D-FINE, transformers models/d_fine/modeling_d_fine.py:168-206): one tap at pixel
// (int(lx * W_l + 0.5), int(ly * H_l + 0.5)) truncated toward zero and clamped into the map, weight = the
// attention weight; corners 1..3 are empty. A NaN coordinate takes pixel 0.
//
// GENERAL = false compiles the reference's case only (P points on every level, bilinear, no mask); kernels are
// instantiated both ways and the launchers pick GENERAL = true only when a mask, per-level point counts, the
// discrete method or accumulation-type locations are in use, so the common path carries none of their cost.
// What a corner-table entry holds for token t: the token (sb = 0; -1 when outside), or its row's byte offset
// t * sb, for the buffer-load gathers (gather_sum_buf), with kOutside, past any buffer of under 2 GB, when outside.
constexpr int kOutside = static_cast<int>(0x80000000u);
__device__ __forceinline__ int corner_ref(bool in, int64_t t, int sb) {
    if (sb == 0) return in ? static_cast<int>(t) : -1;
    return in ? static_cast<int>(t) * sb : kOutside;
}

struct LevelGeom {
    int hl, wl;   // height, width
    int64_t st;   // first token
};
__device__ __forceinline__ LevelGeom level_geom(const Geom& g, int l) {
    return LevelGeom{static_cast<int>(g.shapes[2 * l]), static_cast<int>(g.shapes[2 * l + 1]), g.starts[l]};
}

// The corner rule with the level's geometry already loaded (kernels that sample one level per lane across many rows
// load it once).
template <typename A, bool GENERAL>
__device__ __forceinline__ void corners_lv(A lx, A ly, A w, const LevelGeom& lg, const Geom& g, int64_t row,
                                           Corner<A>* out, int sb = 0) {
    const int hl = lg.hl, wl = lg.wl;
    const int64_t st = lg.st;
    if (GENERAL && g.discrete) {
        const A fx = fmin(fmax(lx * static_cast<A>(wl) + static_cast<A>(0.5), static_cast<A>(-1)), static_cast<A>(wl));
        const A fy = fmin(fmax(ly * static_cast<A>(hl) + static_cast<A>(0.5), static_cast<A>(-1)), static_cast<A>(hl));
        int xi = static_cast<int>(fx), yi = static_cast<int>(fy);  // truncation toward zero
        xi = xi < 0 ? 0 : xi > wl - 1 ? wl - 1 : xi;
        yi = yi < 0 ? 0 : yi > hl - 1 ? hl - 1 : yi;
        const int64_t t = st + static_cast<int64_t>(yi) * wl + xi;
        bool in = wl > 0 && hl > 0 && t >= 0 && t < g.N;
        if (in && g.mask != nullptr) in = g.mask[(row / (static_cast<int64_t>(g.Q) * g.H)) * g.N + t] == 0;
        out[0].tok = corner_ref(in, t, sb);
        out[0].w = in ? w : static_cast<A>(0);
#pragma unroll
        for (int k = 1; k < 4; ++k) out[k] = Corner<A>{corner_ref(false, 0, sb), static_cast<A>(0)};
        return;
    }
    A x = lx * static_cast<A>(wl) - static_cast<A>(0.5);
    A y = ly * static_cast<A>(hl) - static_cast<A>(0.5);
    // fmax returns the non-NaN operand, so a NaN coordinate becomes -2 (outside the map)
    x = fmin(fmax(x, static_cast<A>(-2)), static_cast<A>(wl) + static_cast<A>(1));
    y = fmin(fmax(y, static_cast<A>(-2)), static_cast<A>(hl) + static_cast<A>(1));
    const A xf = floor(x), yf = floor(y);
    const int x0 = static_cast<int>(xf), y0 = static_cast<int>(yf);
    const A fx = x - xf, fy = y - yf;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int dx = k & 1, dy = k >> 1, xi = x0 + dx, yi = y0 + dy;
        const int64_t t = st + static_cast<int64_t>(yi) * wl + xi;
        bool in = xi >= 0 && xi < wl && yi >= 0 && yi < hl && t >= 0 && t < g.N;
        if (GENERAL && in && g.mask != nullptr) in = g.mask[(row / (static_cast<int64_t>(g.Q) * g.H)) * g.N + t] == 0;
        out[k].tok = corner_ref(in, t, sb);
        out[k].w = in ? w * (dx ? fx : static_cast<A>(1) - fx) * (dy ? fy : static_cast<A>(1) - fy)
                      : static_cast<A>(0);
    }
}

template <typename A, bool GENERAL>
__device__ __forceinline__ void corners_at(A lx, A ly, A w, int l, const Geom& g, int64_t row, Corner<A>* out,
                                           int sb = 0) {
    corners_lv<A, GENERAL>(lx, ly, w, level_geom(g, l), g, row, out, sb);
}

// The corners of sample j (j = l * P + p, or the running index over per-level point counts) of row `row`, with the
// location and weight read from loc [rows, LP, 2] and attn [rows, LP] in the element type T (or in the
// accumulation type A when g.loc_acc is set).
template <typename T, typename A, bool GENERAL>
__device__ __forceinline__ void corner4(const T* __restrict__ loc, const T* __restrict__ attn, const Geom& g,
                                        int64_t row, int j, int l, Corner<A>* out, int sb = 0) {
    const int64_t idx = row * g.LP + j;
    A lx, ly, w;
    if (GENERAL && g.loc_acc) {
        const A* la = reinterpret_cast<const A*>(loc);
        lx = la[2 * idx];
        ly = la[2 * idx + 1];
        w = reinterpret_cast<const A*>(attn)[idx];
    } else {
        lx = cvt<A>(loc[2 * idx]);
        ly = cvt<A>(loc[2 * idx + 1]);
        w = cvt<A>(attn[idx]);
    }
    corners_at<A, GENERAL>(lx, ly, w, l, g, row, out, sb);
}
template <typename T, typename A, bool GENERAL>
__device__ __forceinline__ void corner4(const T* __restrict__ loc, const T* __restrict__ attn, const Geom& g,
                                        int64_t row, int j, Corner<A>* out, int sb = 0) {
    corner4<T, A, GENERAL>(loc, attn, g, row, j, GENERAL ? level_of(g, j) : j / g.P, out, sb);
}

// ---- vector loads: Bytes-wide raw loads unpacked to float ------------------------------------------------

template <int Bytes>
struct Raw;
template <>
struct Raw<16> {
    using type = u32x4;
};
template <>
struct Raw<8> {
    using type = u32x2;
};
template <>
struct Raw<4> {
    using type = unsigned;
};
template <>
struct Raw<2> {
    using type = unsigned short;
};

// V elements of T loaded with one V * sizeof(T)-byte load (V * sizeof(T) in {2, 4, 8, 16}).
template <typename T, int V>
struct VecIO {
    static constexpr int kBytes = V * static_cast<int>(sizeof(T));
    using raw_t = typename Raw<kBytes>::type;
    __device__ __forceinline__ static raw_t load(const T* p) { return *reinterpret_cast<const raw_t*>(p); }
    __device__ __forceinline__ static raw_t zero() { return raw_t{}; }
    __device__ __forceinline__ static void unpack(const raw_t& r, float* o) {
        const T* e = reinterpret_cast<const T*>(&r);
#pragma unroll
        for (int i = 0; i < V; ++i) o[i] = static_cast<float>(e[i]);
    }
    __device__ __forceinline__ static void store(T* p, const float* v) {
        raw_t r;
        T* e = reinterpret_cast<T*>(&r);
#pragma unroll
        for (int i = 0; i < V; ++i) e[i] = static_cast<T>(v[i]);
        *reinterpret_cast<raw_t*>(p) = r;
    }
};

// bfloat16 -> float is a 16-bit shift; do it on the packed dwords.
template <int V>
struct VecIO<bf16, V> {
    static constexpr int kBytes = V * 2;
    using raw_t = typename Raw<kBytes>::type;
    __device__ __forceinline__ static raw_t load(const bf16* p) { return *reinterpret_cast<const raw_t*>(p); }
    __device__ __forceinline__ static raw_t zero() { return raw_t{}; }
    __device__ __forceinline__ static void unpack(const raw_t& r, float* o) {
        if constexpr (V == 1) {
            o[0] = __builtin_bit_cast(float, static_cast<unsigned>(r) << 16);
        } else {
            const unsigned* u = reinterpret_cast<const unsigned*>(&r);
#pragma unroll
            for (int i = 0; i < V / 2; ++i) {
                o[2 * i] = __builtin_bit_cast(float, u[i] << 16);
                o[2 * i + 1] = __builtin_bit_cast(float, u[i] & 0xffff0000u);
            }
        }
    }
    __device__ __forceinline__ static void store(bf16* p, const float* v) {
        raw_t r;
        bf16* e = reinterpret_cast<bf16*>(&r);
#pragma unroll
        for (int i = 0; i < V; ++i) e[i] = static_cast<bf16>(v[i]);
        *reinterpret_cast<raw_t*>(p) = r;
    }
};

// Weighted sum of gathered rows: acc[0..V) += w_s * row(tok_s)[0..V) for corners s = first, first + step, ...
// below S, where row(t) = col + t * stride; ws += w_s. Loads are issued NB at a time before any of them is
// consumed, so NB row reads per lane are in flight together. Corners outside the map (tok < 0) and the padding
// slots of a last, partial batch read row 0 (always valid) and contribute exactly 0; full batches skip the slot
// check (the gather loops are bound by the instructions they issue).
template <typename T, int V, int NB>
__device__ __forceinline__ void gather_sum(const Corner<float>* __restrict__ cr, int S, int first, int step,
                                           const T* __restrict__ col, size_t stride, float* acc, float& ws) {
    using IO = VecIO<T, V>;
    auto batch = [&](int s0, bool check) {
        typename IO::raw_t raw[NB];
        float w[NB];
        bool in[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int s = s0 + u * step;
            const Corner<float> c = !check || s < S ? cr[s] : Corner<float>{-1, 0.f};
            w[u] = c.w;
            in[u] = c.tok >= 0;
            raw[u] = IO::load(col + static_cast<size_t>(in[u] ? c.tok : 0) * stride);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const typename IO::raw_t r = in[u] ? raw[u] : IO::zero();
            float v[V];
            IO::unpack(r, v);
            ws += w[u];
#pragma unroll
            for (int i = 0; i < V; ++i) acc[i] = fmaf(w[u], v[i], acc[i]);
        }
    };
    int s0 = first;
    for (; s0 + step * (NB - 1) < S; s0 += step * NB) batch(s0, false);
    if (s0 < S) batch(s0, true);
}

// A raw buffer over [base, base + bytes), bytes < 2^31: loads past the end return zeros (gfx9 range checking).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
template <typename R>
__device__ __forceinline__ R buffer_load(__amdgpu_buffer_rsrc_t rsrc, unsigned off) {
    if constexpr (sizeof(R) == 16)
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b128(rsrc, static_cast<int>(off), 0, 0));
    else if constexpr (sizeof(R) == 8)
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b64(rsrc, static_cast<int>(off), 0, 0));
    else
        return __builtin_bit_cast(R, __builtin_amdgcn_raw_buffer_load_b32(rsrc, static_cast<int>(off), 0, 0));
}

// gather_sum over a corner table of byte offsets (corner_ref with sb = the row stride in bytes): row s is at
// byte lane_off + off_s of the buffer, and an outside corner's offset (kOutside + lane_off) lies past its end, so
// the load itself returns zeros: per corner one add instead of a multiply, a 64-bit address and a select of the
// loaded data. V * sizeof(T) must be 4, 8 or 16 bytes.
template <typename T, int V, int NB>
__device__ __forceinline__ void gather_sum_buf(const Corner<float>* __restrict__ cr, int S, int first, int step,
                                               __amdgpu_buffer_rsrc_t rsrc, unsigned lane_off, float* acc, float& ws) {
    using IO = VecIO<T, V>;
    using R = typename IO::raw_t;
    static_assert(sizeof(R) == 4 || sizeof(R) == 8 || sizeof(R) == 16, "buffer load width");
    auto batch = [&](int s0, bool check) {
        R raw[NB];
        float w[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int s = s0 + u * step;
            const Corner<float> c = !check || s < S ? cr[s] : Corner<float>{kOutside, 0.f};
            w[u] = c.w;
            raw[u] = buffer_load<R>(rsrc, static_cast<unsigned>(c.tok) + lane_off);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            float v[V];
            IO::unpack(raw[u], v);
            ws += w[u];
#pragma unroll
            for (int i = 0; i < V; ++i) acc[i] = fmaf(w[u], v[i], acc[i]);
        }
    };
    int s0 = first;
    for (; s0 + step * (NB - 1) < S; s0 += step * NB) batch(s0, false);
    if (s0 < S) batch(s0, true);
}

// ---- cross-lane ----------------------------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

// Value of `v` in lane (lane ^ mask) of the same wavefront.
__device__ __forceinline__ float xor_lane(float v, int mask) {
    const int src = (lane_id() ^ mask) << 2;
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(src, __builtin_bit_cast(int, v)));
}
__device__ __forceinline__ double xor_lane(double v, int mask) {
    const int src = (lane_id() ^ mask) << 2;
    const long long u = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(u));
    const int hi = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(u >> 32));
    return __builtin_bit_cast(double, (static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

// Sum over the 64 lanes of a wavefront (every lane receives the total).
template <typename A>
__device__ __forceinline__ A wave_sum(A v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += xor_lane(v, m);
    return v;
}

}  // namespace td
