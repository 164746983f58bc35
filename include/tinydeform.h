/*
 * tinydeform.h -- C ABI of the MI355X (gfx950) value-projection + multi-scale deformable attention library
 * (libtinydeform.so, built from marearts_tinydeform_amd/csrc).
 *
 * Every entry point takes plain device pointers, element counts and a hipStream_t passed as void*.
 * The library never allocates or frees device memory and never synchronises: callers own every buffer,
 * kernels run asynchronously on the given stream, and each call may be captured in a HIP graph.
 * The level geometry (spatial_shapes, level_start_index) is read on the device, never on the host.
 *
 * Tensor layouts (all row-major, contiguous, one element type `dtype` for every floating tensor):
 *   memory              [B, N, C]
 *   value_weight        [H*D, C]          (an nn.Linear weight)
 *   value_bias          [H*D] or NULL
 *   value               [B, N, H*D]       (memory @ value_weight^T + value_bias)
 *   spatial_shapes      [L, 2] int64      (height, width) per level, tokens laid out level by level
 *   level_start_index   [L] int64         first token of each level
 *   sampling_locations  [B, Q, H, L, P, 2] (x, y) normalised to [0, 1]
 *   attention_weights   [B, Q, H, L, P]
 *   out                 [B, Q, H*D]
 *
 * Return value: TD_OK (0) or a negative TD_E* code; td_last_error() then describes the failure
 * (thread-local, valid until the next call on the same thread).
 */
#ifndef TINYDEFORM_H
#define TINYDEFORM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types: codes for the `dtype` argument */
#define TD_F32 0
#define TD_F16 1
#define TD_BF16 2
#define TD_F64 3

/* error codes */
#define TD_OK 0
#define TD_E_ARG -1    /* invalid shape, limit or pointer (the same cases the reference rejects) */
#define TD_E_DTYPE -2  /* unknown dtype code */
#define TD_E_LAUNCH -3 /* the HIP runtime refused a kernel launch */
#define TD_E_WORKSPACE -4 /* td_layer_fused_forward: this problem needs loc_out and attn_out (see there);
                              td_weight_grad: the workspace is smaller than td_weight_grad_workspace() */

/* limits shared with the reference operator (csrc/ma_deform_fused.cu:26-28) */
#define TD_MAX_LEVEL_POINTS 64 /* L * P */
#define TD_MAX_CHANNELS 8192   /* C, fused mode */

/* Library version, e.g. 100 for 0.1.0. */
int td_version(void);

/* Message for the last non-zero return on this thread ("" if none). */
const char* td_last_error(void);

/*
 * Fused mode: out[b,q,h*D+d] = W[h*D+d] . (sum_s w_s memory[b,t_s]) + bias[h*D+d] * sum_s w_s,
 * s over the L*P*4 bilinear corners inside the map (align_corners=False, zero padding).
 * Replaces the pybind entry `fused_forward(memory, weight, bias, spatial_shapes, level_start_index,
 * sampling_locations, attention_weights)` of the reference (csrc/ma_deform_fused.cu:291-325).
 * dtype: TD_F32, TD_F16, TD_BF16 (float32 accumulation) or TD_F64 (float64 accumulation).
 * Limits: L*P <= 64, C <= 8192, N <= INT32_MAX, B*Q*H <= INT32_MAX.
 */
int td_fused_forward(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                     const int64_t* spatial_shapes, const int64_t* level_start_index,
                     const void* sampling_locations, const void* attention_weights, void* out,
                     int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H, int64_t D, int64_t L, int64_t P,
                     void* stream);

/*
 * Sampling on projected values (the second half of project mode):
 * out[b,q,h*D+d] = sum_s w_s value[b,t_s,h*D+d].
 * Replaces the pybind entry `sample_forward(value, heads, spatial_shapes, level_start_index,
 * sampling_locations, attention_weights)` of the reference (csrc/ma_deform_fused.cu:327-350).
 */
int td_sample_forward(int dtype, const void* value, const int64_t* spatial_shapes,
                      const int64_t* level_start_index, const void* sampling_locations,
                      const void* attention_weights, void* out, int64_t B, int64_t Q, int64_t N, int64_t H,
                      int64_t D, int64_t L, int64_t P, void* stream);

/*
 * td_fused_forward / td_sample_forward with a value padding mask: padding_mask is a device array of B*N bytes,
 * non-zero marking a padded token whose value row is zero (value.masked_fill(padding_mask[..., None], 0) after the
 * projection, as Deformable-DETR decoders do); NULL means no mask. A corner on a padded token contributes nothing,
 * bias share included. No counterpart in the reference, which does not support a padding mask (README.md:62);
 * needed by batches of images padded to one size.
 */
int td_fused_forward_masked(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                            const int64_t* spatial_shapes, const int64_t* level_start_index,
                            const void* sampling_locations, const void* attention_weights,
                            const uint8_t* padding_mask, void* out, int64_t B, int64_t Q, int64_t N, int64_t C,
                            int64_t H, int64_t D, int64_t L, int64_t P, void* stream);

int td_sample_forward_masked(int dtype, const void* value, const int64_t* spatial_shapes,
                             const int64_t* level_start_index, const void* sampling_locations,
                             const void* attention_weights, const uint8_t* padding_mask, void* out, int64_t B,
                             int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P, void* stream);

/*
 * The two halves of td_project_forward with the head-major value layout, for callers that keep the projected values
 * between calls. td_value_proj_heads: value [B, H, N, D] = memory [B, N, C] @ value_weight[H * D, C]^T + bias, float32
 * accumulation, one rounding; D * element size must be a multiple of 16 bytes. td_sample_forward_heads: sampling of
 * such a value into out [B, Q, H, D], arguments as td_project_forward. No counterpart in the reference, whose value
 * is always [B, N, H * D] (marearts_tinydeform/__init__.py:77): with D = 32 16-bit elements a head row is 64 bytes, and
 * head-major places the two corners of a bilinear pair (x0, x0 + 1) in one 128-byte run.
 */
int td_value_proj_heads(int dtype, const void* memory, const void* value_weight, const void* value_bias, void* value,
                        int64_t B, int64_t N, int64_t C, int64_t H, int64_t D, void* stream);
int td_sample_forward_heads(int dtype, const void* value, const int64_t* spatial_shapes,
                            const int64_t* level_start_index, const void* sampling_locations,
                            const void* attention_weights, const uint8_t* padding_mask, int loc_acc, void* out,
                            int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P, void* stream);

/*
 * Project mode in one call: value_ws = memory @ value_weight^T + value_bias on the library's GEMM, then sampling of
 * value_ws into out [B, Q, H, D]. value_ws is caller-provided device memory of B * N * H * D elements of dtype that
 * holds the projected values afterwards in a layout the library picks (head-major [B, H, N, D] when a head row is 64
 * bytes or less, else [B, N, H * D]), so callers treat it as scratch. loc_acc = 1: sampling_locations and
 * attention_weights are float32 (float64 for TD_F64), as td_layer_prologue writes them; 0: dtype. padding_mask as in
 * td_sample_forward_masked. Replaces the reference's F.linear + _C.sample_forward pair of mode='project'
 * (marearts_tinydeform/__init__.py:77-80, csrc/ma_deform_fused.cu:327-350).
 */
int td_project_forward(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                       const int64_t* spatial_shapes, const int64_t* level_start_index,
                       const void* sampling_locations, const void* attention_weights, const uint8_t* padding_mask,
                       int loc_acc, void* value_ws, void* out, int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H,
                       int64_t D, int64_t L, int64_t P, void* stream);

/*
 * td_project_forward without the value_ws workspace: the projected values go to a static device array of
 * TD_NOALLOC_SCRATCH_BYTES per GPU instead, so the call allocates nothing (no hipMalloc, no allocating library
 * routine). No counterpart in the reference; for callers that cannot allocate: code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc. A problem whose projected values (B*N*H*D elements of dtype) exceed
 * the array is refused with TD_E_ARG (td_project_forward with a workspace takes it). Every call on one GPU shares
 * that GPU's array, so calls that overlap on one GPU (other streams, other host threads) race; the stream's device
 * must be the current device (else TD_E_ARG). Same results as td_project_forward, bit for bit.
 */
#define TD_NOALLOC_SCRATCH_BYTES 67108864 /* 64 MiB per GPU */
int td_project_forward_noalloc(int dtype, const void* memory, const void* value_weight, const void* value_bias,
                               const int64_t* spatial_shapes, const int64_t* level_start_index,
                               const void* sampling_locations, const void* attention_weights,
                               const uint8_t* padding_mask, int loc_acc, void* out, int64_t B, int64_t Q, int64_t N,
                               int64_t C, int64_t H, int64_t D, int64_t L, int64_t P, void* stream);

/*
 * Sampling with per-level point counts and a choice of sampling method (the deformable attention core of D-FINE:
 * transformers models/d_fine/modeling_d_fine.py:150-216, multi_scale_deformable_attention_v2). Level l has
 * points_per_level[l] samples (a host array of L entries, sum <= 64), so sampling_locations is
 * [B, Q, H, sum, 2] and attention_weights [B, Q, H, sum]. discrete = 0: bilinear with zero padding
 * (align_corners=False); discrete = 1: the nearest-pixel rule of D-FINE's "discrete" method. padding_mask as in
 * td_sample_forward_masked (NULL for none). No counterpart in the reference (README.md:62 lists discrete sampling
 * as unsupported); needed by D-FINE / RT-DETRv2-style decoders, which have no value projection.
 */
int td_sample_forward_v2(int dtype, const void* value, const int64_t* spatial_shapes,
                         const int64_t* level_start_index, const void* sampling_locations,
                         const void* attention_weights, const uint8_t* padding_mask, void* out, int64_t B, int64_t Q,
                         int64_t N, int64_t H, int64_t D, int64_t L, const int64_t* points_per_level, int discrete,
                         void* stream);

/*
 * Decoder-layer entries: the query side of a deformable-attention layer computed on the device, restating
 * HF transformers RTDetrMultiscaleDeformableAttention.forward (models/rt_detr/modeling_rt_detr.py:673-713):
 *   x          = query[b,q] (+ position[b,q])                                  query, position: [B, Q, Cq]
 *   offsets    = x @ offsets_weight^T + offsets_bias      offsets_weight [H*L*P*2, Cq], viewed [H, L, P, 2]
 *   attention  = softmax over L*P of (x @ attn_weight^T + attn_bias), per head; attn_weight [H*L*P, Cq]
 *   location   = ref[b,q,l] + offsets / (W_l, H_l)                        ref_dim = 2
 *              = ref[b,q,l,0:2] + offsets / P * ref[b,q,l,2:4] * 0.5      ref_dim = 4 (box centre and size)
 * reference_points is [B, Q, ref_levels, ref_dim] with ref_levels 1 (shared by every level) or L. Biases and
 * position may be NULL. Locations and weights are computed in float32 (float64 for TD_F64) and never rounded to
 * dtype. No counterpart in the reference, whose operator starts from ready locations and weights; these fuse the
 * producers of those inputs into the operator (the sampling-offset and attention projections, the softmax and the
 * reference-point arithmetic), so they need no HBM round trip and no separate launches.
 */

/*
 * Query prologue alone: writes loc_out [B, Q, H, L, P, 2] and attn_out [B, Q, H, L, P], both float32 (float64 for
 * TD_F64). Used ahead of td_layer_sample_forward in project mode.
 */
int td_layer_prologue(int dtype, const void* query, const void* position, const void* reference_points,
                      int64_t ref_levels, int64_t ref_dim, const void* offsets_weight, const void* offsets_bias,
                      const void* attn_weight, const void* attn_bias, const int64_t* spatial_shapes, void* loc_out,
                      void* attn_out, int64_t B, int64_t Q, int64_t Cq, int64_t H, int64_t L, int64_t P,
                      void* stream);

/*
 * Fused layer: the query prologue inside the fused-mode kernel (td_fused_forward_masked with the locations and
 * weights computed in-kernel). out [B, Q, H*D] as td_fused_forward; padding_mask as td_fused_forward_masked.
 * loc_out / attn_out (float32, float64 for TD_F64; NULL for none) receive the locations and weights when given.
 * Problems the in-kernel prologue does not take run the standalone prologue into loc_out / attn_out and then the
 * fused kernel: for those both buffers are required, and without them the call returns TD_E_WORKSPACE having
 * launched nothing. They are: TD_F64; C or Cq not a multiple of 16 bytes; rows not 16-byte aligned; query
 * projections of B * Q * H * 3 * L * P * Cq >= 8e8 multiply-adds (they run on the GEMM); and projection weights of
 * more than 256 KB per head (3 * L * P * Cq elements), or more than 64 KB per head with B * Q >= 200.
 */
int td_layer_fused_forward(int dtype, const void* query, const void* position, const void* reference_points,
                           int64_t ref_levels, int64_t ref_dim, const void* offsets_weight, const void* offsets_bias,
                           const void* attn_weight, const void* attn_bias, const void* memory,
                           const void* value_weight, const void* value_bias, const int64_t* spatial_shapes,
                           const int64_t* level_start_index, const uint8_t* padding_mask, void* out, void* loc_out,
                           void* attn_out, int64_t B, int64_t Q, int64_t N, int64_t Cq, int64_t C, int64_t H,
                           int64_t D, int64_t L, int64_t P, void* stream);

/*
 * td_sample_forward_masked with locations and weights in float32 (float64 for TD_F64), as td_layer_prologue
 * writes them: the second half of the layer's project mode.
 */
int td_layer_sample_forward(int dtype, const void* value, const int64_t* spatial_shapes,
                            const int64_t* level_start_index, const void* loc, const void* attn,
                            const uint8_t* padding_mask, void* out, int64_t B, int64_t Q, int64_t N, int64_t H,
                            int64_t D, int64_t L, int64_t P, void* stream);

/*
 * Value projection (the first half of project mode): value[M, NO] = memory[M, K] @ weight[NO, K]^T + bias[NO],
 * float32 accumulation, one rounding to dtype. M = B*N tokens, K = C, NO = H*D.
 * Replaces the reference's F.linear(memory, value_weight, value_bias) call (marearts_tinydeform/__init__.py:77).
 */
int td_value_proj(int dtype, const void* memory, const void* weight, const void* bias, void* value, int64_t M,
                  int64_t K, int64_t NO, void* stream);

/*
 * Which value-projection kernel td_value_proj (head_major_N = 0) or td_value_proj_heads (head_major_N = N, with H
 * heads) launches for these operands: the tile variant number, 0 for the generic VALU kernel, or a negative TD_E*
 * code. The pointers are only inspected for their alignment, never read, so any address of the right alignment will
 * do. No counterpart in the reference (it calls F.linear); for tests and tuning, which check that every kernel the
 * size rule can pick has a parity case.
 */
int td_value_proj_plan(int dtype, const void* memory, const void* weight, const void* bias, const void* value,
                       int64_t M, int64_t K, int64_t NO, int64_t head_major_N, int64_t H);

/*
 * Launch shapes the size rules of td_fused_forward and td_sample_forward pick for these sizes, written to plan[8]
 * without launching anything or reading memory (aligned = 1: operands on 16-byte boundaries, the usual case). No
 * counterpart in the reference; the auto selector's cost model (choose_mode) is built on them, as the kernels' time
 * follows the rows their busiest CUs hold.
 *   td_fused_plan:  plan = {kernel (0 vector, 1 generic, -1 none), workgroups, wavefronts per workgroup, rows per
 *                   workgroup, balanced slices per head (0: query tiles), rows of the largest workgroup, corner
 *                   groups per row, corner loads in flight per lane}
 *   td_sample_plan: plan = {workgroups (-1 in plan[0]: none), wavefronts per workgroup, rows per workgroup, corner
 *                   groups per row, elements per load, 1 when rows go in (b, h, q) order, corner loads in flight per
 *                   lane, 0}; head_major = 1 for the [B, H, N, D] value layout of td_sample_forward_heads.
 */
int td_fused_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H, int64_t D, int64_t L, int64_t P,
                  int aligned, int64_t* plan);
int td_sample_plan(int dtype, int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P,
                   int head_major, int aligned, int64_t* plan);

/*
 * Backward (training). No counterpart in the reference, whose operator is inference only (README.md:61); these are
 * the gradients of its reference computation (reference.py:13-40: value = memory . W^T + b, then bilinear
 * grid_sample with zero padding, align_corners=False, weighted by the attention), for callers that train through
 * the operator. The caller owns every buffer, workspaces included.
 */

/*
 * Sampling half: given grad_out [B, Q, H*D] and the forward's value, locations and weights,
 *   grad_value_acc [B, N, H*D]  float32 (float64 for TD_F64): zeroed, then accumulated (the gradient of value);
 *   grad_value     [B, N, H*D]  dtype, or NULL: grad_value_acc rounded to dtype (may be grad_value_acc itself for
 *                               TD_F32 / TD_F64). For TD_F16 / TD_BF16 with grad_value given, decoder shapes with
 *                               many corners (2^18 or more) may have grad_value written directly, by binning the
 *                               corners by token, with grad_value_acc used as scratch only: its contents are then
 *                               unspecified, so read the value gradient from grad_value;
 *   grad_loc [B, Q, H, L, P, 2], grad_attn [B, Q, H, L, P]: dtype.
 * padding_mask as in td_sample_forward_masked. Limits as td_sample_forward, and D <= 256.
 */
int td_sample_backward(int dtype, const void* value, const int64_t* spatial_shapes, const int64_t* level_start_index,
                       const void* sampling_locations, const void* attention_weights, const uint8_t* padding_mask,
                       const void* grad_out, void* grad_value_acc, void* grad_value, void* grad_loc, void* grad_attn,
                       int64_t B, int64_t Q, int64_t N, int64_t H, int64_t D, int64_t L, int64_t P, void* stream);

/*
 * Projection, input side: grad_memory[M, C] = grad_value[M, HD] . value_weight[HD, C] on the library's GEMM.
 * weight_t: a workspace of HD*C elements of dtype, which receives value_weight^T.
 */
int td_input_grad(int dtype, const void* grad_value, const void* value_weight, void* weight_t, void* grad_memory,
                  int64_t M, int64_t HD, int64_t C, void* stream);

/* Bytes of workspace td_weight_grad needs for these sizes. */
int64_t td_weight_grad_workspace(int dtype, int64_t M, int64_t HD, int64_t C);

/*
 * Projection, weight side: grad_weight[HD, C] = grad_value[M, HD]^T . memory[M, C] and grad_bias[HD] = the column
 * sums of grad_value (NULL: not computed). Split over the M tokens, with per-split float32 (float64) partials in
 * the workspace summed in a fixed order, so the result is the same on every run.
 */
int td_weight_grad(int dtype, const void* grad_value, const void* memory, void* grad_weight, void* grad_bias,
                   int64_t M, int64_t HD, int64_t C, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * td_input_grad and td_weight_grad of the same grad_value in one call, with the same arguments, results and
 * workspace (td_weight_grad_workspace; TD_E_WORKSPACE before anything is launched when it is smaller). Where the
 * input gradient's GEMM takes the small-grid tiles (below about 14000 tokens of 256 channels in 16 bits) its tiles
 * and the weight gradient's share one launch; no counterpart in the reference, whose operator is inference only.
 * There, and where the input gradient takes the streaming GEMM (C = 256, HD = 128 or 256, many tokens), in 16 bits
 * with C a multiple of 8 and value_weight 16-byte aligned, the GEMM reads value_weight as stored (LDS transpose
 * reads) and weight_t is left unwritten; otherwise weight_t receives value_weight^T as in td_input_grad.
 */
int td_input_weight_grad(int dtype, const void* grad_value, const void* value_weight, void* weight_t,
                         const void* memory, void* grad_memory, void* grad_weight, void* grad_bias, int64_t M,
                         int64_t HD, int64_t C, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Measurement kernels. No counterpart in the reference and no part of the operator: the benchmark uses them to
 * calibrate what it reports.
 *
 * td_probe_empty: `launches` launches of a kernel that does nothing (one wavefront). Traced, it gives the duration
 * a kernel tracer reports for a dispatch with no work.
 *
 * td_probe_gather: one launch of `workgroups` workgroups of `waves` wavefronts that read randomly chosen rows of
 * buf [bytes] (below 2 GB), row_bytes / 16 lanes per row by 16-byte buffer loads, 8 loads in flight per lane,
 * loads_per_lane (a multiple of 8) per lane in all: the gather kernels' access pattern, at the rate the CUs can
 * receive such rows. sink: `workgroups` 32-bit words, written only when the loaded data xor to 0x5a5a5a5a (never
 * for a zero buffer).
 */
int td_probe_empty(int64_t launches, void* stream);
/*
 * td_probe_atomic: one launch of `workgroups` workgroups of 256 threads in groups of `lanes` lanes (16, 32 or 64);
 * each group adds 1.0f, lane by lane, to `adds_per_group` chunks of lanes * 4 bytes of buf [bytes] (float), chosen by
 * a hash of the step (random != 0) or in sequence: the float atomics of the value-gradient scatter, at the rate the
 * GPU applies them.
 */
int td_probe_atomic(void* buf, int64_t bytes, int64_t lanes, int64_t adds_per_group, int64_t workgroups, int random,
                    void* stream);
int td_probe_gather(const void* buf, int64_t bytes, int64_t row_bytes, int64_t loads_per_lane, int64_t workgroups,
                    int64_t waves, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TINYDEFORM_H */
