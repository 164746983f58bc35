// C ABI of libtinydeform.so (declared in include/tinydeform.h): argument checks, then the kernel launchers.
// The checks restate the reference's size and limit checks (csrc/ma_deform_fused.cu:236-266, 298-308, 333);
// dtype and device agreement between tensors is the caller's job (the Python layer checks it).
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "../../include/tinydeform.h"
#include "td_internal.h"

namespace td {

namespace {
thread_local std::string g_last_error;

__global__ void zero_kernel(unsigned* p, int64_t words) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride) p[i] = 0u;
}
// 16 bytes per store
__global__ void zero16_kernel(u32x4* p, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        p[i] = u32x4{0u, 0u, 0u, 0u};
}
__global__ void zero_bytes_kernel(unsigned char* p, int64_t bytes) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < bytes) p[i] = 0;
}
}  // namespace

int set_error(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

int launch_zero(void* out, int64_t bytes, hipStream_t stream) {
    if (bytes <= 0) return 0;
    if (reinterpret_cast<uintptr_t>(out) % 16 == 0 && bytes % 16 == 0) {
        const int64_t n = bytes / 16;
        int64_t blocks = (n + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(zero16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                           static_cast<u32x4*>(out), n);
    } else if (reinterpret_cast<uintptr_t>(out) % 4 == 0 && bytes % 4 == 0) {
        const int64_t words = bytes / 4;
        int64_t blocks = (words + 255) / 256;
        if (blocks > 4096) blocks = 4096;
        hipLaunchKernelGGL(zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream,
                           static_cast<unsigned*>(out), words);
    } else {
        hipLaunchKernelGGL(zero_bytes_kernel, dim3(static_cast<unsigned>((bytes + 255) / 256)), dim3(256), 0, stream,
                           static_cast<unsigned char*>(out), bytes);
    }
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : set_error(TD_E_LAUNCH, "zero fill launch failed: %s", hipGetErrorString(e));
}

namespace {

constexpr int64_t kInt32Max = 2147483647;

bool dtype_ok(int dtype) { return dtype == TD_F32 || dtype == TD_F16 || dtype == TD_BF16 || dtype == TD_F64; }

// Sizes and limits common to fused and sample mode (reference csrc/ma_deform_fused.cu:236-266).
int check_geometry(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P,
                   const int64_t* shapes, const int64_t* starts, const void* loc, const void* attn, const void* out) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (B < 0 || Q < 0 || N < 0 || H < 0 || D < 0 || L < 0 || P < 0)
        return set_error(TD_E_ARG, "sizes must be non-negative");
    if (N > kInt32Max) return set_error(TD_E_ARG, "too many memory tokens");
    if (H <= 0) return set_error(TD_E_ARG, "need at least one head");
    if (L * P > kMaxLevelPoints) return set_error(TD_E_ARG, "levels x points must be <= %d", kMaxLevelPoints);
    if (B * Q * H > kInt32Max) return set_error(TD_E_ARG, "too many (batch, query, head) rows");
    if (H * D > kInt32Max) return set_error(TD_E_ARG, "too many output channels");
    if (B * Q * H * D > 0) {
        if (out == nullptr || loc == nullptr || attn == nullptr || (L > 0 && (shapes == nullptr || starts == nullptr)))
            return set_error(TD_E_ARG, "null pointer argument");
    }
    return TD_OK;
}

}  // namespace
}  // namespace td

using namespace td;

extern "C" int td_version(void) { return 100; }

extern "C" const char* td_last_error(void) { return g_last_error.c_str(); }

namespace {

// Sizes a plan query accepts: those the forward entries accept (check_geometry without the pointers).
int check_plan_sizes(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P,
                     int64_t* plan) {
    g_last_error.clear();
    if (plan == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    for (int i = 0; i < 8; ++i) plan[i] = 0;
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (B < 0 || Q < 0 || N < 0 || H <= 0 || D < 0 || L < 0 || P < 0) return set_error(TD_E_ARG, "invalid sizes");
    if (N > kInt32Max || L * P > kMaxLevelPoints || B * Q * H > kInt32Max || H * D > kInt32Max)
        return set_error(TD_E_ARG, "sizes beyond the operator's limits");
    return TD_OK;
}

// Stand-ins for the buffers of a plan query: never read. `aligned` = 0 gives addresses off 16-byte alignment.
const void* plan_ptr(int aligned) { return reinterpret_cast<const void*>(aligned ? 0x10000 : 0x10002); }

}  // namespace

extern "C" int td_fused_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H, int64_t D, int64_t L,
                             int64_t P, int aligned, int64_t* plan) {
    int rc = check_plan_sizes(dtype, B, Q, N, H, D, L, P, plan);
    if (rc != TD_OK) return rc;
    if (C < 0 || C > kMaxChannels) return set_error(TD_E_ARG, "channels must be <= %d", kMaxChannels);
    if (B * Q * H * D == 0 || N == 0 || L * P == 0) {
        plan[0] = -1;  // no kernel: an empty output, or a zero fill
        return TD_OK;
    }
    Geom g{nullptr, nullptr, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N), static_cast<int>(H),
           static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), nullptr};
    set_levels(g, nullptr);
    LaunchPlan lp;
    FusedTune tune;
    tune.plan = &lp;
    const void* ptr = plan_ptr(aligned);
    rc = launch_fused(dtype, ptr, ptr, nullptr, g, static_cast<int>(C), ptr, ptr, const_cast<void*>(ptr), nullptr,
                      tune);
    if (rc != 0) return rc;
    for (int i = 0; i < 8; ++i) plan[i] = lp.v[i];
    return TD_OK;
}

extern "C" int td_sample_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P,
                              int head_major, int aligned, int64_t* plan) {
    int rc = check_plan_sizes(dtype, B, Q, N, H, D, L, P, plan);
    if (rc != TD_OK) return rc;
    if (B * Q * H * D == 0 || N == 0 || L * P == 0) {
        plan[0] = -1;
        return TD_OK;
    }
    Geom g{nullptr, nullptr, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N), static_cast<int>(H),
           static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), nullptr};
    set_levels(g, nullptr);
    g.value_hm = head_major ? 1 : 0;
    LaunchPlan lp;
    SampleTune tune;
    tune.plan = &lp;
    const void* ptr = plan_ptr(aligned);
    rc = launch_sample(dtype, ptr, g, ptr, ptr, const_cast<void*>(ptr), nullptr, tune);
    if (rc != 0) return rc;
    for (int i = 0; i < 8; ++i) plan[i] = lp.v[i];
    return TD_OK;
}

extern "C" int td_fused_forward_masked(int dtype, const void* memory, const void* value_weight,
                                       const void* value_bias, const int64_t* spatial_shapes,
                                       const int64_t* level_start_index, const void* sampling_locations,
                                       const void* attention_weights, const uint8_t* padding_mask, void* out,
                                       int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H, int64_t D, int64_t L,
                                       int64_t P, void* stream) {
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, out);
    if (rc != TD_OK) return rc;
    if (C < 0 || C > kMaxChannels) return set_error(TD_E_ARG, "channels must be <= %d", kMaxChannels);
    if (B * N * C > 0 && memory == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    if (H * D * C > 0 && value_weight == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H * D == 0) return TD_OK;
    const int64_t bytes = B * Q * H * D * elem_size(dtype);
    // no tokens: every corner is outside, so the output is exactly zero (the bias share included)
    if (N == 0 || L * P == 0) return launch_zero(out, bytes, s);
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), padding_mask};
    set_levels(g, nullptr);
    FusedTune tune;
    return launch_fused(dtype, memory, value_weight, value_bias, g, static_cast<int>(C), sampling_locations,
                        attention_weights, out, s, tune);
}

extern "C" int td_sample_forward_masked(int dtype, const void* value, const int64_t* spatial_shapes,
                                        const int64_t* level_start_index, const void* sampling_locations,
                                        const void* attention_weights, const uint8_t* padding_mask, void* out,
                                        int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P,
                                        void* stream) {
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, out);
    if (rc != TD_OK) return rc;
    if (B * N * H * D > 0 && value == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H * D == 0) return TD_OK;
    const int64_t bytes = B * Q * H * D * elem_size(dtype);
    if (N == 0 || L * P == 0) return launch_zero(out, bytes, s);
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), padding_mask};
    set_levels(g, nullptr);
    SampleTune tune;
    return launch_sample(dtype, value, g, sampling_locations, attention_weights, out, s, tune);
}

extern "C" int td_sample_forward_v2(int dtype, const void* value, const int64_t* spatial_shapes,
                                    const int64_t* level_start_index, const void* sampling_locations,
                                    const void* attention_weights, const uint8_t* padding_mask, void* out, int64_t B,
                                    int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L,
                                    const int64_t* points_per_level, int discrete, void* stream) {
    g_last_error.clear();
    if (L < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (L > kMaxLevelPoints) return set_error(TD_E_ARG, "levels x points must be <= %d", kMaxLevelPoints);
    if (L > 0 && points_per_level == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    if (discrete != 0 && discrete != 1) return set_error(TD_E_ARG, "method must be 0 (bilinear) or 1 (discrete)");
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), 1, padding_mask};
    if (!set_levels(g, points_per_level))
        return set_error(TD_E_ARG, "levels x points must be <= %d (and point counts non-negative)", kMaxLevelPoints);
    g.discrete = discrete;
    // the shared checks see the samples of a row as L levels of one point each plus the total
    int rc = check_geometry(dtype, B, Q, N, H, D, 1, g.LP, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, out);
    if (rc != TD_OK) return rc;
    if (B * N * H * D > 0 && value == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H * D == 0) return TD_OK;
    const int64_t bytes = B * Q * H * D * elem_size(dtype);
    if (N == 0 || g.LP == 0) return launch_zero(out, bytes, s);
    SampleTune tune;
    return launch_sample(dtype, value, g, sampling_locations, attention_weights, out, s, tune);
}

namespace {

// Query-side checks of the layer entries.
int check_layer(int64_t Cq, int64_t ref_levels, int64_t ref_dim, int64_t L, int64_t P, const void* query,
                const void* ref, const void* off_w, const void* aw_w, int64_t rows) {
    if (Cq < 0 || Cq > kMaxChannels) return set_error(TD_E_ARG, "query channels must be <= %d", kMaxChannels);
    if (ref_dim != 2 && ref_dim != 4) return set_error(TD_E_ARG, "reference points must have 2 or 4 coordinates");
    if (ref_levels != 1 && ref_levels != L)
        return set_error(TD_E_ARG, "reference points must have 1 or L (= %lld) levels", static_cast<long long>(L));
    if (rows > 0 && L * P > 0 && (query == nullptr || ref == nullptr || (Cq > 0 && (off_w == nullptr || aw_w == nullptr))))
        return set_error(TD_E_ARG, "null pointer argument");
    return TD_OK;
}

LayerArgs layer_args(const void* query, const void* position, const void* ref, int64_t ref_levels, int64_t ref_dim,
                     const void* off_w, const void* off_b, const void* aw_w, const void* aw_b, void* loc_out,
                     void* attn_out, int64_t Cq) {
    LayerArgs la;
    la.query = query;
    la.pos = position;
    la.ref = ref;
    la.off_w = off_w;
    la.off_b = off_b;
    la.aw_w = aw_w;
    la.aw_b = aw_b;
    la.loc_out = loc_out;
    la.attn_out = attn_out;
    la.Cq = static_cast<int>(Cq);
    la.RL = static_cast<int>(ref_levels);
    la.RD = static_cast<int>(ref_dim);
    return la;
}

}  // namespace

extern "C" int td_layer_prologue(int dtype, const void* query, const void* position, const void* reference_points,
                                 int64_t ref_levels, int64_t ref_dim, const void* offsets_weight,
                                 const void* offsets_bias, const void* attn_weight, const void* attn_bias,
                                 const int64_t* spatial_shapes, void* loc_out, void* attn_out, int64_t B, int64_t Q,
                                 int64_t Cq, int64_t H, int64_t L, int64_t P, void* stream) {
    // the level starts are not needed here: pass the shapes in their place for the shared checks
    int rc = check_geometry(dtype, B, Q, 0, H, 1, L, P, spatial_shapes, spatial_shapes, loc_out, attn_out, loc_out);
    if (rc != TD_OK) return rc;
    rc = check_layer(Cq, ref_levels, ref_dim, L, P, query, reference_points, offsets_weight, attn_weight, B * Q * H);
    if (rc != TD_OK) return rc;
    if (B * Q * H * L * P == 0) return TD_OK;
    Geom g{spatial_shapes, spatial_shapes, static_cast<int>(B), static_cast<int>(Q), 0, static_cast<int>(H), 1,
           static_cast<int>(L), static_cast<int>(P)};
    set_levels(g, nullptr);
    const LayerArgs la = layer_args(query, position, reference_points, ref_levels, ref_dim, offsets_weight,
                                    offsets_bias, attn_weight, attn_bias, loc_out, attn_out, Cq);
    return launch_prologue(dtype, la, g, static_cast<hipStream_t>(stream));
}

// Whether the fused layer kernel computes the query prologue itself. It streams a head's projection weights
// (3 L P Cq elements) once per 16 queries, so large weights per head, and projections big enough for the GEMM
// route, go to the standalone prologue and then the fused kernel. Measured on MI355X (layer, fused mode, µs):
// C = 1024, 16 heads x 4 levels x 16 points (393 KB per head), 100 query rows 120.7 -> 99.0; C = 512, 16 x 4 x 16
// (196 KB), 300 rows 114.0 -> 98.9 but 100 rows 57.6 against 61.7; C = 1024, 16 x 3 x 4 (74 KB), 300 rows
// 97.2 -> 83.9; up to 37 KB per head (RT-DETR, DINO, C = 512 with 12 samples) either way alike.
static bool layer_prologue_in_kernel(int dtype, const Geom& g, int64_t Cq) {
    if (prologue_wants_gemm(dtype, g, Cq)) return false;
    const double per_head = 3.0 * g.LP * static_cast<double>(Cq) * elem_size(dtype);
    const int64_t rows = static_cast<int64_t>(g.B) * g.Q;
    return !(per_head > 256 * 1024 || (per_head > 64 * 1024 && rows >= 200));
}

extern "C" int td_layer_fused_forward(int dtype, const void* query, const void* position,
                                      const void* reference_points, int64_t ref_levels, int64_t ref_dim,
                                      const void* offsets_weight, const void* offsets_bias, const void* attn_weight,
                                      const void* attn_bias, const void* memory, const void* value_weight,
                                      const void* value_bias, const int64_t* spatial_shapes,
                                      const int64_t* level_start_index, const uint8_t* padding_mask, void* out,
                                      void* loc_out, void* attn_out, int64_t B, int64_t Q, int64_t N, int64_t Cq,
                                      int64_t C, int64_t H, int64_t D, int64_t L, int64_t P, void* stream) {
    // the shared checks see the query and the reference points in place of ready locations and weights
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, query, reference_points,
                            out);
    if (rc != TD_OK) return rc;
    if (C < 0 || C > kMaxChannels) return set_error(TD_E_ARG, "channels must be <= %d", kMaxChannels);
    if (B * N * C > 0 && memory == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    if (H * D * C > 0 && value_weight == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    rc = check_layer(Cq, ref_levels, ref_dim, L, P, query, reference_points, offsets_weight, attn_weight, B * Q * H);
    if (rc != TD_OK) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H == 0) return TD_OK;
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), padding_mask};
    set_levels(g, nullptr);
    const LayerArgs la = layer_args(query, position, reference_points, ref_levels, ref_dim, offsets_weight,
                                    offsets_bias, attn_weight, attn_bias, loc_out, attn_out, Cq);
    const bool want_prologue = L * P > 0 && (loc_out != nullptr || attn_out != nullptr);
    if (D == 0 || N == 0 || L * P == 0) {
        // nothing to gather: the output is exactly zero (bias share included); locations still go out if asked
        if (want_prologue) {
            if (loc_out == nullptr || attn_out == nullptr)
                return set_error(TD_E_WORKSPACE, "layer: give both loc_out and attn_out, or neither");
            rc = launch_prologue(dtype, la, g, s);
            if (rc != TD_OK) return rc;
        }
        return launch_zero(out, B * Q * H * D * elem_size(dtype), s);
    }
    FusedTune tune;
    if (layer_prologue_in_kernel(dtype, g, Cq)) {
        rc = launch_fused(dtype, memory, value_weight, value_bias, g, static_cast<int>(C), nullptr, nullptr, out, s,
                          tune, &la);
        if (rc != 1) return rc;
    }
    // the in-kernel prologue does not take this problem: standalone prologue, then the fused kernel on its output
    if (loc_out == nullptr || attn_out == nullptr)
        return set_error(TD_E_WORKSPACE,
                         "layer: float64, rows that are not 16-byte multiples or not 16-byte aligned, or large query "
                         "projections need loc_out and attn_out");
    rc = launch_prologue(dtype, la, g, s);
    if (rc != TD_OK) return rc;
    g.loc_acc = 1;
    return launch_fused(dtype, memory, value_weight, value_bias, g, static_cast<int>(C), loc_out, attn_out, out, s,
                        tune);
}

extern "C" int td_layer_sample_forward(int dtype, const void* value, const int64_t* spatial_shapes,
                                       const int64_t* level_start_index, const void* loc, const void* attn,
                                       const uint8_t* padding_mask, void* out, int64_t B, int64_t Q, int64_t N,
                                       int64_t H, int64_t D, int64_t L, int64_t P, void* stream) {
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, loc, attn, out);
    if (rc != TD_OK) return rc;
    if (B * N * H * D > 0 && value == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H * D == 0) return TD_OK;
    if (N == 0 || L * P == 0) return launch_zero(out, B * Q * H * D * elem_size(dtype), s);
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), padding_mask};
    set_levels(g, nullptr);
    g.loc_acc = 1;
    SampleTune tune;
    return launch_sample(dtype, value, g, loc, attn, out, s, tune);
}

namespace {
// Head-major value when a head row is 64 bytes or less: the sampler's bilinear pairs (x0, x0 + 1) are then one
// contiguous run instead of two rows H * D apart
bool head_major_pays(int dtype, int64_t D) {
    const int64_t row_bytes = D * elem_size(dtype);
    return dtype != TD_F64 && row_bytes <= 64 && row_bytes % 16 == 0;
}

int check_proj_sizes(int dtype, int64_t M, int64_t K, int64_t NO) {
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (M < 0 || K < 0 || NO < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (M > kInt32Max || K > kInt32Max || NO > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    return TD_OK;
}

int sample_heads(int dtype, const void* value, const int64_t* spatial_shapes, const int64_t* level_start_index,
                 const void* loc, const void* attn, const uint8_t* padding_mask, int loc_acc, void* out, int64_t B,
                 int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P, hipStream_t s) {
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), padding_mask};
    set_levels(g, nullptr);
    g.loc_acc = loc_acc;
    g.value_hm = 1;
    SampleTune tune;
    return launch_sample(dtype, value, g, loc, attn, out, s, tune);
}
}  // namespace

extern "C" int td_value_proj_heads(int dtype, const void* memory, const void* weight, const void* bias, void* value,
                                   int64_t B, int64_t N, int64_t C, int64_t H, int64_t D, void* stream) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (B < 0 || N < 0 || C < 0 || H <= 0 || D <= 0) return set_error(TD_E_ARG, "need B, N, C >= 0 and H, D >= 1");
    const int rc = check_proj_sizes(dtype, B * N, C, H * D);
    if (rc != TD_OK) return rc;
    if ((D * elem_size(dtype)) % 16 != 0) return set_error(TD_E_ARG, "head row must be a multiple of 16 bytes");
    if (B * N == 0) return TD_OK;
    if (value == nullptr || (C > 0 && (memory == nullptr || weight == nullptr)))
        return set_error(TD_E_ARG, "null pointer argument");
    return launch_value_proj(dtype, memory, weight, bias, value, B * N, C, H * D, static_cast<hipStream_t>(stream),
                             static_cast<int>(N), static_cast<int>(H));
}

extern "C" int td_sample_forward_heads(int dtype, const void* value, const int64_t* spatial_shapes,
                                       const int64_t* level_start_index, const void* sampling_locations,
                                       const void* attention_weights, const uint8_t* padding_mask, int loc_acc,
                                       void* out, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L,
                                       int64_t P, void* stream) {
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, out);
    if (rc != TD_OK) return rc;
    if (loc_acc != 0 && loc_acc != 1) return set_error(TD_E_ARG, "loc_acc must be 0 or 1");
    if (B * N * H * D > 0 && value == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H * D == 0) return TD_OK;
    if (N == 0 || L * P == 0) return launch_zero(out, B * Q * H * D * elem_size(dtype), s);
    return sample_heads(dtype, value, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                        padding_mask, loc_acc, out, B, Q, N, H, D, L, P, s);
}

namespace td {

int project_forward(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                    const int64_t* spatial_shapes, const int64_t* level_start_index, const void* sampling_locations,
                    const void* attention_weights, const uint8_t* padding_mask, int loc_acc, void* value_ws,
                    int64_t value_ws_bytes, void* out, int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H,
                    int64_t D, int64_t L, int64_t P, void* stream) {
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, out);
    if (rc != TD_OK) return rc;
    if (loc_acc != 0 && loc_acc != 1) return set_error(TD_E_ARG, "loc_acc must be 0 or 1");
    if (C < 0 || C > kInt32Max || B * N > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (B * Q * H * D == 0) return TD_OK;
    if (N == 0 || L * P == 0) return launch_zero(out, B * Q * H * D * elem_size(dtype), s);
    if (value_ws_bytes >= 0 && B * N * H * D * elem_size(dtype) > value_ws_bytes)
        return set_error(TD_E_ARG, "project: the projected values need %lld bytes, more than the %lld available",
                         static_cast<long long>(B * N * H * D * elem_size(dtype)),
                         static_cast<long long>(value_ws_bytes));
    if (value_ws == nullptr || (C > 0 && (memory == nullptr || value_weight == nullptr)))
        return set_error(TD_E_ARG, "null pointer argument");
    const bool hm = head_major_pays(dtype, D);
    rc = launch_value_proj(dtype, memory, value_weight, value_bias, value_ws, B * N, C, H * D, s,
                           hm ? static_cast<int>(N) : 0, hm ? static_cast<int>(H) : 0);
    if (rc != TD_OK) return rc;
    if (hm)
        return sample_heads(dtype, value_ws, spatial_shapes, level_start_index, sampling_locations, attention_weights,
                            padding_mask, loc_acc, out, B, Q, N, H, D, L, P, s);
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P), padding_mask};
    set_levels(g, nullptr);
    g.loc_acc = loc_acc;
    SampleTune tune;
    return launch_sample(dtype, value_ws, g, sampling_locations, attention_weights, out, s, tune);
}

}  // namespace td

extern "C" int td_project_forward(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                                  const int64_t* spatial_shapes, const int64_t* level_start_index,
                                  const void* sampling_locations, const void* attention_weights,
                                  const uint8_t* padding_mask, int loc_acc, void* value_ws, void* out, int64_t B,
                                  int64_t Q, int64_t N, int64_t C, int64_t H, int64_t D, int64_t L, int64_t P,
                                  void* stream) {
    return project_forward(dtype, memory, value_weight, value_bias, spatial_shapes, level_start_index,
                           sampling_locations, attention_weights, padding_mask, loc_acc, value_ws, -1, out, B, Q, N, C,
                           H, D, L, P, stream);
}

extern "C" int td_fused_forward(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                                const int64_t* spatial_shapes, const int64_t* level_start_index,
                                const void* sampling_locations, const void* attention_weights, void* out, int64_t B,
                                int64_t Q, int64_t N, int64_t C, int64_t H, int64_t D, int64_t L, int64_t P,
                                void* stream) {
    return td_fused_forward_masked(dtype, memory, value_weight, value_bias, spatial_shapes, level_start_index,
                                   sampling_locations, attention_weights, nullptr, out, B, Q, N, C, H, D, L, P, stream);
}

extern "C" int td_sample_forward(int dtype, const void* value, const int64_t* spatial_shapes,
                                 const int64_t* level_start_index, const void* sampling_locations,
                                 const void* attention_weights, void* out, int64_t B, int64_t Q, int64_t N,
                                 int64_t H, int64_t D, int64_t L, int64_t P, void* stream) {
    return td_sample_forward_masked(dtype, value, spatial_shapes, level_start_index, sampling_locations,
                                    attention_weights, nullptr, out, B, Q, N, H, D, L, P, stream);
}

extern "C" int td_value_proj(int dtype, const void* memory, const void* weight, const void* bias, void* value,
                             int64_t M, int64_t K, int64_t NO, void* stream) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (M < 0 || K < 0 || NO < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (M > kInt32Max || K > kInt32Max || NO > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    if (M * NO == 0) return TD_OK;
    if (value == nullptr || (K > 0 && (memory == nullptr || weight == nullptr)))
        return set_error(TD_E_ARG, "null pointer argument");
    return launch_value_proj(dtype, memory, weight, bias, value, M, K, NO, static_cast<hipStream_t>(stream));
}

extern "C" int td_value_proj_plan(int dtype, const void* memory, const void* weight, const void* bias,
                                  const void* value, int64_t M, int64_t K, int64_t NO, int64_t head_major_N,
                                  int64_t H) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (M < 0 || K < 0 || NO < 0 || head_major_N < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (M > kInt32Max || K > kInt32Max || NO > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    if (head_major_N > 0 && (H <= 0 || NO % H != 0 || M % head_major_N != 0))
        return set_error(TD_E_ARG, "head-major output needs H dividing NO and N dividing M");
    return value_proj_plan(dtype, memory, weight, bias, value, M, K, NO, static_cast<int>(head_major_N),
                           static_cast<int>(head_major_N > 0 ? H : 0));
}

extern "C" int td_sample_backward(int dtype, const void* value, const int64_t* spatial_shapes,
                                  const int64_t* level_start_index, const void* sampling_locations,
                                  const void* attention_weights, const uint8_t* padding_mask, const void* grad_out,
                                  void* grad_value_acc, void* grad_value, void* grad_loc, void* grad_attn, int64_t B,
                                  int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P, void* stream) {
    int rc = check_geometry(dtype, B, Q, N, H, D, L, P, spatial_shapes, level_start_index, sampling_locations,
                            attention_weights, grad_loc);
    if (rc != TD_OK) return rc;
    if (B * N * H * D > 0 && grad_value_acc == nullptr) return set_error(TD_E_ARG, "null pointer argument");
    if (B * Q * H * L * P > 0 && (value == nullptr || grad_out == nullptr || grad_attn == nullptr))
        return set_error(TD_E_ARG, "null pointer argument");
    if (D > 256) return set_error(TD_E_ARG, "sample backward: head dim must be <= 256");
    Geom g{spatial_shapes, level_start_index, static_cast<int>(B), static_cast<int>(Q), static_cast<int>(N),
           static_cast<int>(H), static_cast<int>(D), static_cast<int>(L), static_cast<int>(P)};
    g.mask = padding_mask;
    set_levels(g, nullptr);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    bool direct = false;
    rc = launch_sample_backward(dtype, value, g, sampling_locations, attention_weights, grad_out, grad_value_acc,
                                grad_value == grad_value_acc ? nullptr : grad_value, grad_loc, grad_attn, s, &direct);
    if (rc != TD_OK || direct || grad_value == nullptr || grad_value == grad_value_acc) return rc;
    return launch_convert(dtype, grad_value_acc, grad_value, B * N * H * D, s);
}

extern "C" int td_input_grad(int dtype, const void* grad_value, const void* value_weight, void* weight_t,
                             void* grad_memory, int64_t M, int64_t HD, int64_t C, void* stream) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (M < 0 || HD < 0 || C < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (M > kInt32Max || HD > kInt32Max || C > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    if (M * C == 0) return TD_OK;
    if (grad_memory == nullptr || (HD > 0 && (grad_value == nullptr || value_weight == nullptr || weight_t == nullptr)))
        return set_error(TD_E_ARG, "null pointer argument");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int rc = launch_transpose(dtype, value_weight, weight_t, HD, C, s);
    if (rc != TD_OK) return rc;
    return launch_value_proj(dtype, grad_value, weight_t, nullptr, grad_memory, M, HD, C, s);
}

extern "C" int64_t td_weight_grad_workspace(int dtype, int64_t M, int64_t HD, int64_t C) {
    int splits = 1, chunk = 32;
    int64_t bytes = 0;
    if (M < 0 || HD < 0 || C < 0) return 0;
    wgrad_plan(M, HD, C, dtype, &splits, &chunk, &bytes);
    return bytes;
}

extern "C" int td_input_weight_grad(int dtype, const void* grad_value, const void* value_weight, void* weight_t,
                                    const void* memory, void* grad_memory, void* grad_weight, void* grad_bias,
                                    int64_t M, int64_t HD, int64_t C, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (M < 0 || HD < 0 || C < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (M > kInt32Max || HD > kInt32Max || C > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    if (M == 0 || HD == 0 || C == 0) {  // the two entries' own handling of empty sizes
        int rc = td_input_grad(dtype, grad_value, value_weight, weight_t, grad_memory, M, HD, C, stream);
        if (rc != TD_OK) return rc;
        return td_weight_grad(dtype, grad_value, memory, grad_weight, grad_bias, M, HD, C, workspace, workspace_bytes,
                              stream);
    }
    if (grad_value == nullptr || value_weight == nullptr || weight_t == nullptr || memory == nullptr ||
        grad_memory == nullptr || grad_weight == nullptr)
        return set_error(TD_E_ARG, "null pointer argument");
    const int64_t need = td_weight_grad_workspace(dtype, M, HD, C);
    if (workspace == nullptr || workspace_bytes < need)
        return set_error(TD_E_WORKSPACE, "weight gradient: workspace of %lld bytes needed, %lld given",
                         static_cast<long long>(need), static_cast<long long>(workspace_bytes));
    return launch_input_weight_grad(dtype, grad_value, value_weight, weight_t, memory, grad_memory, grad_weight,
                                    grad_bias, M, HD, C, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

extern "C" int td_weight_grad(int dtype, const void* grad_value, const void* memory, void* grad_weight,
                              void* grad_bias, int64_t M, int64_t HD, int64_t C, void* workspace,
                              int64_t workspace_bytes, void* stream) {
    g_last_error.clear();
    if (!dtype_ok(dtype)) return set_error(TD_E_DTYPE, "unknown dtype code %d", dtype);
    if (M < 0 || HD < 0 || C < 0) return set_error(TD_E_ARG, "sizes must be non-negative");
    if (M > kInt32Max || HD > kInt32Max || C > kInt32Max) return set_error(TD_E_ARG, "GEMM size exceeds int32");
    if (HD * C == 0 && (grad_bias == nullptr || HD == 0)) return TD_OK;
    if (grad_weight == nullptr || (M > 0 && (grad_value == nullptr || memory == nullptr)))
        return set_error(TD_E_ARG, "null pointer argument");
    return launch_wgrad(dtype, grad_value, memory, grad_weight, grad_bias, M, HD, C, workspace, workspace_bytes,
                        static_cast<hipStream_t>(stream));
}
