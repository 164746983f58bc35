// Project mode without a caller workspace: td_project_forward_noalloc keeps the projected values in a file-scope
// device array, so the call allocates nothing (for callers that cannot allocate: code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc).
//
// Each GPU the library runs on holds its own copy of `scratch` (TD_NOALLOC_SCRATCH_BYTES) until the process ends.
// Host code never passes `scratch` itself to a kernel (in host code the name is a host-side stand-in, not a device
// address): the first call on a device resolves the array's device address there with hipGetSymbolAddress, with
// that device current, and keeps it per device. Every call on one GPU shares that GPU's array and overwrites every
// byte of it that it reads, so nothing needs clearing between calls; calls that overlap on one GPU (concurrent
// streams, other host threads) race on it.
#include <mutex>

#include "../../include/tinydeform.h"
#include "td_internal.h"

namespace td {
namespace {

static_assert(TD_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
__device__ __align__(256) unsigned char scratch[TD_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the stream's device, resolved once per device with that device current. The
// stream's device must be the current one: hipGetSymbolAddress answers for the current device, and the kernels run
// on the stream's, so a mismatch would hand one GPU's address to another's kernels. Returns 0 with *out set, or the
// error code it recorded.
int device_scratch(hipStream_t stream, void** out) {
    int dev = -1, sdev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error(TD_E_LAUNCH, "noalloc: no current HIP device: %s", hipGetErrorString(e));
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess)
        return set_error(TD_E_ARG, "noalloc: cannot tell the stream's device: %s", hipGetErrorString(e));
    if (sdev != dev)
        return set_error(TD_E_ARG, "noalloc: the stream belongs to device %d but device %d is current (make the "
                         "stream's device current)", sdev, dev);
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(TD_E_ARG, "noalloc: device %d is beyond the %d this library serves", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return set_error(TD_E_LAUNCH, "noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s",
                             dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace td

using namespace td;

extern "C" int td_project_forward_noalloc(int dtype, const void* memory, const void* value_weight,
                                          const void* value_bias, const int64_t* spatial_shapes,
                                          const int64_t* level_start_index, const void* sampling_locations,
                                          const void* attention_weights, const uint8_t* padding_mask, int loc_acc,
                                          void* out, int64_t B, int64_t Q, int64_t N, int64_t C, int64_t H,
                                          int64_t D, int64_t L, int64_t P, void* stream) {
    // the size limit first, so that an oversized call is refused before anything else happens
    if (B > 0 && N > 0 && H > 0 && D > 0 && dtype >= TD_F32 && dtype <= TD_F64 &&
        B * N * H * D > TD_NOALLOC_SCRATCH_BYTES / elem_size(dtype))
        return set_error(TD_E_ARG,
                         "project_forward_noalloc: the projected values need %lld bytes, more than the %lld-byte "
                         "scratch array (use td_project_forward with a workspace)",
                         static_cast<long long>(B * N * H * D * elem_size(dtype)),
                         static_cast<long long>(TD_NOALLOC_SCRATCH_BYTES));
    void* ws = nullptr;
    const int rc = device_scratch(static_cast<hipStream_t>(stream), &ws);
    if (rc != 0) return rc;
    return project_forward(dtype, memory, value_weight, value_bias, spatial_shapes, level_start_index,
                           sampling_locations, attention_weights, padding_mask, loc_acc, ws, TD_NOALLOC_SCRATCH_BYTES,
                           out, B, Q, N, C, H, D, L, P, stream);
}
