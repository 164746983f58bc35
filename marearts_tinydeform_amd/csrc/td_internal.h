// Host-side declarations shared by the kernel translation units and the C ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "td_common.h"
#include "td_prologue.h"

namespace td {

enum Dtype { kF32 = 0, kF16 = 1, kBF16 = 2, kF64 = 3 };

inline int elem_size(int dtype) { return dtype == kF64 ? 8 : dtype == kF32 ? 4 : 2; }

// The launch shape a launcher chose, reported instead of launching when a tune struct's `plan` is set (the size
// rules of td_fused_plan / td_sample_plan, for the auto selector's cost model). No memory is read.
struct LaunchPlan {
    int64_t v[8] = {};
};

// Launch shape of the fused kernels; zero fields are chosen by the launcher.
struct FusedTune {
    int qt = 0;     // query rows per workgroup (1..16)
    int sg = 0;     // corner split per row (power of two)
    int waves = 0;  // wavefronts per workgroup (4 or 8)
    int generic = 0;  // 1 forces the generic kernel
    // set: fill it (kernel: 0 vector, 1 generic; workgroups; wavefronts per workgroup; rows per workgroup; balanced
    // slices per head, 0 for query tiles; rows of the largest workgroup; corner groups per row; corner loads in
    // flight per lane) and return 0 without launching
    LaunchPlan* plan = nullptr;
};

// Launch shape of the sampling kernel; zero fields are chosen by the launcher.
struct SampleTune {
    int sg = 0;
    int waves = 0;
    int vec = 0;  // elements per load
    // set: fill it (workgroups; wavefronts per workgroup; rows per workgroup; corner groups per row; elements per
    // load; 1 for rows in (b, h, q) order; corner loads in flight per lane) and return 0 without launching
    LaunchPlan* plan = nullptr;
};

// Compute units of the current device (256 on MI355X), cached per device.
int cu_count();

// Lets kernel `fn` launch with up to `bytes` of dynamic LDS (above the default 64 KB; MI355X has 160 KB per CU) on the
// current device. The attribute is set once per device: `done` (one per kernel) holds a bit per device already set.
inline hipError_t allow_dynamic_lds(const void* fn, int bytes, std::atomic<uint64_t>& done) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const uint64_t bit = uint64_t{1} << (dev & 63);
    if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
    e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
    return e;
}

// Every launcher returns 0, or a negative TD_E* code after recording a message with set_error.
int set_error(int code, const char* fmt, ...);

// layer != null: the decoder-layer kernel, whose query prologue computes locations and weights in-kernel (loc and
// attn are then unused). Returns 1, launching nothing, when the vector kernel cannot take a layer problem.
int launch_fused(int dtype, const void* mem, const void* w, const void* bias, const Geom& g, int C,
                 const void* loc, const void* attn, void* out, hipStream_t stream, const FusedTune& tune,
                 const LayerArgs* layer = nullptr);

// Standalone query prologue: locations [B, Q, H, L, P, 2] and attention weights [B, Q, H, L, P] in the
// accumulation type (layer.loc_out / layer.attn_out, both required).
// route: 0 picks by size, 1 forces the single-kernel prologue, 2 the GEMM route (projections on the GEMM, then an
// in-place finalize; falls back to the single kernel for float64 or unaligned operands).
int launch_prologue(int dtype, const LayerArgs& layer, const Geom& g, hipStream_t stream, int route = 0);

// Whether the query projections are large enough for the GEMM route (8e8 multiply-adds; not float64). The fused
// layer kernel streams a head's projection weights once per 16 queries, so such problems run the standalone
// prologue and then the fused kernel instead.
bool prologue_wants_gemm(int dtype, const Geom& g, int64_t Cq);

int launch_sample(int dtype, const void* value, const Geom& g, const void* loc, const void* attn, void* out,
                  hipStream_t stream, const SampleTune& tune);

// The kernel is picked by size and operand alignment (value_proj_plan). hm_N > 0: c is head-major
// [M / hm_N, hm_H, hm_N, NO / hm_H] instead of [M, NO] (rows are b * hm_N + t); the head width NO / hm_H must be a
// multiple of 16 bytes.
int launch_value_proj(int dtype, const void* a, const void* w, const void* bias, void* c, int64_t M, int64_t K,
                      int64_t NO, hipStream_t stream, int hm_N = 0, int hm_H = 0);
// The tile variant launch_value_proj runs for these operands (0: the generic kernel); reads no memory.
int value_proj_plan(int dtype, const void* a, const void* w, const void* bias, const void* c, int64_t M, int64_t K,
                    int64_t NO, int hm_N = 0, int hm_H = 0);

// Projection in float32 for the layer prologue: c[M, NO] = a[M, K] . w[NO, K]^T (+ a2[M, K] . w^T) + bias, float32
// accumulation, stored unrounded; a2 may be null. 16/32-bit operands with K a multiple of 16 bytes and 16-byte
// aligned a, a2, w and c. Returns 1, launching nothing, when the operands do not qualify.
int launch_proj_f32(int dtype, const void* a, const void* a2, const void* w, const void* bias, float* c, int64_t M,
                    int64_t K, int64_t NO, hipStream_t stream);
// Two such projections of the same rows in one launch (td_gemm_dma.hip): c_j[M, no_j] = x . w_j^T (+ x2 . w_j^T)
// + b_j, j = 0, 1; x2, b0 and b1 may be null. 16-bit operands, K % 64 == 0, no_j % 4 == 0, 16-byte aligned x, x2,
// w_j and c_j, 8-byte aligned biases. With fin and g (the layer prologue: c_0 = raw offsets, c_1 = raw logits) and
// L * P a power of two from 4 to 64, the kernel also finalizes them into locations and softmax weights, as
// layer_finalize_kernel does, and returns 2. Returns 0 when it launched the raw projections, and 1, launching
// nothing, when the operands do not qualify.
int launch_proj_f32_pair(int dtype, const void* x, const void* x2, const void* w0, const void* b0, float* c0,
                         int64_t no0, const void* w1, const void* b1, float* c1, int64_t no1, int64_t M, int64_t K,
                         hipStream_t stream, const LayerArgs* fin = nullptr, const Geom* g = nullptr);

int launch_zero(void* out, int64_t bytes, hipStream_t stream);

// Project mode (td_project_forward) with the projected values in value_ws; value_ws_bytes >= 0 bounds the bytes
// they may take (an error beyond it), -1 leaves the size to the caller.
int project_forward(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                    const int64_t* spatial_shapes, const int64_t* level_start_index, const void* sampling_locations,
                    const void* attention_weights, const uint8_t* padding_mask, int loc_acc, void* value_ws,
                    int64_t value_ws_bytes, void* out, int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H,
                    int64_t D, int64_t L, int64_t P, void* stream);

// Backward (td_backward.hip). grad_value: [B, N, H*D] in the accumulation type, zeroed and accumulated here;
// grad_loc / grad_attn in the element type (the accumulation type with g.loc_acc).
// grad_value: the float32 (float64) accumulator; grad_value_t: the element-type gradient or NULL. *direct is set
// when grad_value_t was written directly (the accumulator then held scratch), else the caller rounds the accumulator.
int launch_sample_backward(int dtype, const void* value, const Geom& g, const void* loc, const void* attn,
                           const void* grad_out, void* grad_value, void* grad_value_t, void* grad_loc, void* grad_attn,
                           hipStream_t stream, bool* direct);
// dst[i] = src[i] rounded from the accumulation type to dtype
int launch_convert(int dtype, const void* src_acc, void* dst, int64_t n, hipStream_t stream);
// dst [Cc, R] = src [R, Cc]^T
int launch_transpose(int dtype, const void* src, void* dst, int64_t R, int64_t Cc, hipStream_t stream);
// weight / bias gradient split over tokens: partials in the workspace, summed in a fixed order
void wgrad_plan(int64_t M, int64_t NO, int64_t K, int dtype, int* splits, int* chunk, int64_t* ws_bytes);
// with_gemm: a GEMM run in the same launch on the 64 x 64 two-stage tiles (launch_input_weight_grad); gemm_wt: its W
// is given as stored, [K, NO] (16-bit types only)
struct GemmParams;
int launch_wgrad(int dtype, const void* G, const void* X, void* gw, void* gb, int64_t M, int64_t NO, int64_t K,
                 void* workspace, int64_t ws_bytes, hipStream_t stream, const GemmParams* with_gemm = nullptr,
                 bool gemm_wt = false);
int launch_input_weight_grad(int dtype, const void* G, const void* W, void* Wt, const void* X, void* gm, void* gw,
                             void* gb, int64_t M, int64_t HD, int64_t C, void* workspace, int64_t ws_bytes,
                             hipStream_t stream);

}  // namespace td
