// Measurement kernels (not part of the operator; bench.py uses them to put the operator's figures in context).
//
// probe_empty_kernel   does nothing. A graph of such launches, traced, gives what a kernel tracer reports for a
//                      dispatch with no work: the dispatch's own fixed cost as the tracer sees it, which the traced
//                      durations of the real kernels also contain.
// probe_gather_kernel  reads randomly chosen rows of a buffer the way the gather kernels do (raw 16-byte buffer
//                      loads, row_bytes / 16 lanes per row, NB loads in flight per lane, consumed together), on every
//                      CU at once. With a buffer of the memory tensor's size it measures how fast the CUs receive
//                      such rows from L2 (and from HBM for what L2 misses): the ceiling of the fused kernel's gather
//                      phase, which moves mostly L2-resident rows.
// probe_atomic_kernel  float atomic adds the way the value-gradient scatter issues them: groups of 16, 32 or 64 lanes,
//                      each group adding to one chunk of 64, 128 or 256 bytes, the chunks chosen by a hash of the
//                      group's step (as the corners of unrelated queries) or in sequence: the rate the L2s apply
//                      such atomics at, the ceiling of the backward's scatter.
#include "../../include/tinydeform.h"
#include "td_internal.h"

namespace td {
namespace {

__global__ void probe_empty_kernel() {}

struct ProbeParams {
    const void* buf;
    int bytes;       // buffer bytes, below 2^31
    unsigned rows;   // whole rows in the buffer
    unsigned row_bytes;
    int lanes_log2;  // log2(row_bytes / 16): the lanes that read one row
    int iters;       // batches of NB loads per lane
    unsigned* sink;  // one word per workgroup, written only if the loaded data xor to a value that zeros never give
};

template <int NB>
__global__ __launch_bounds__(512) void probe_gather_kernel(ProbeParams p) {
    const unsigned tid = blockIdx.x * blockDim.x + threadIdx.x;
    const unsigned ch = tid & ((1u << p.lanes_log2) - 1u);
    // one linear congruential stream per row group (the lanes of a row share it, so they read the same row); the
    // row is the top bits of the state scaled to the row count
    unsigned x = (tid >> p.lanes_log2) * 2654435761u + 0x9e3779b9u;
    const __amdgpu_buffer_rsrc_t rsrc = buffer_of(p.buf, p.bytes);
    const unsigned lane_off = ch * 16u;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (int it = 0; it < p.iters; ++it) {
        u32x4 v[NB];
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            x = x * 1664525u + 1013904223u;
            const unsigned row = __umulhi(x, p.rows);
            v[u] = buffer_load<u32x4>(rsrc, row * p.row_bytes + lane_off);
        }
#pragma unroll
        for (int u = 0; u < NB; ++u) acc ^= v[u];
    }
    const unsigned r = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (r == 0x5a5a5a5au) p.sink[blockIdx.x] = r;  // keeps the loads; a zero buffer never takes it
}

__global__ __launch_bounds__(256) void probe_atomic_kernel(float* __restrict__ buf, unsigned chunks, int lanes_log2,
                                                           unsigned per_group, int random) {
    const unsigned tid = blockIdx.x * blockDim.x + threadIdx.x;
    const unsigned lane = tid & ((1u << lanes_log2) - 1u), group = tid >> lanes_log2;
    for (unsigned i = 0; i < per_group; ++i) {
        const unsigned k = group * per_group + i;
        unsigned c;
        if (random) {
            unsigned x = k * 2654435761u;
            x ^= x >> 15;
            x *= 2246822519u;
            x ^= x >> 13;
            c = __umulhi(x, chunks);
        } else {
            c = k % chunks;
        }
        atomicAdd(buf + (static_cast<size_t>(c) << lanes_log2) + lane, 1.0f);
    }
}

}  // namespace
}  // namespace td

using namespace td;

extern "C" int td_probe_empty(int64_t launches, void* stream) {
    if (launches < 0) return set_error(TD_E_ARG, "probe_empty: launches must be >= 0");
    for (int64_t i = 0; i < launches; ++i) {
        hipLaunchKernelGGL(probe_empty_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream));
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return set_error(TD_E_LAUNCH, "probe_empty: %s", hipGetErrorString(e));
    }
    return 0;
}

extern "C" int td_probe_atomic(void* buf, int64_t bytes, int64_t lanes, int64_t adds_per_group, int64_t workgroups,
                               int random, void* stream) {
    if (buf == nullptr) return set_error(TD_E_ARG, "probe_atomic: null buffer");
    if (lanes != 16 && lanes != 32 && lanes != 64) return set_error(TD_E_ARG, "probe_atomic: lanes must be 16, 32 or 64");
    const int64_t chunks = bytes / (4 * lanes);
    if (chunks < 1 || chunks >= (int64_t{1} << 31))
        return set_error(TD_E_ARG, "probe_atomic: the buffer must hold 1 .. 2^31 - 1 chunks of %lld bytes",
                         static_cast<long long>(4 * lanes));
    if (workgroups < 1 || workgroups > (int64_t{1} << 20) || adds_per_group < 1 || adds_per_group > (int64_t{1} << 16))
        return set_error(TD_E_ARG, "probe_atomic: 1 .. 2^20 workgroups, 1 .. 2^16 adds per lane group");
    int lanes_log2 = 0;
    while ((int64_t{1} << lanes_log2) < lanes) ++lanes_log2;
    hipLaunchKernelGGL(probe_atomic_kernel, dim3(static_cast<unsigned>(workgroups)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<float*>(buf), static_cast<unsigned>(chunks),
                       lanes_log2, static_cast<unsigned>(adds_per_group), random ? 1 : 0);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(TD_E_LAUNCH, "probe_atomic: %s", hipGetErrorString(e));
    return 0;
}

extern "C" int td_probe_gather(const void* buf, int64_t bytes, int64_t row_bytes, int64_t loads_per_lane,
                               int64_t workgroups, int64_t waves, void* sink, void* stream) {
    if (buf == nullptr || sink == nullptr) return set_error(TD_E_ARG, "probe_gather: null buffer");
    if (bytes <= 0 || bytes >= (int64_t{1} << 31))
        return set_error(TD_E_ARG, "probe_gather: the buffer must be 1 byte .. 2 GB - 1 (got %lld)",
                         static_cast<long long>(bytes));
    if (row_bytes < 16 || row_bytes > 1024 || (row_bytes & (row_bytes - 1)) != 0 || row_bytes > bytes)
        return set_error(TD_E_ARG, "probe_gather: row_bytes must be a power of two from 16 to 1024, within the buffer");
    if (workgroups < 1 || workgroups > (int64_t{1} << 20) || (waves != 1 && waves != 2 && waves != 4 && waves != 8))
        return set_error(TD_E_ARG, "probe_gather: 1 .. 2^20 workgroups of 1, 2, 4 or 8 wavefronts");
    if (loads_per_lane < 8 || loads_per_lane % 8 != 0 || loads_per_lane > (int64_t{1} << 24))
        return set_error(TD_E_ARG, "probe_gather: loads_per_lane must be a multiple of 8 up to 2^24");
    ProbeParams p;
    p.buf = buf;
    p.bytes = static_cast<int>(bytes);
    p.rows = static_cast<unsigned>(bytes / row_bytes);
    p.row_bytes = static_cast<unsigned>(row_bytes);
    p.lanes_log2 = 0;
    while ((16 << p.lanes_log2) < row_bytes) ++p.lanes_log2;
    p.iters = static_cast<int>(loads_per_lane / 8);
    p.sink = static_cast<unsigned*>(sink);
    hipLaunchKernelGGL(probe_gather_kernel<8>, dim3(static_cast<unsigned>(workgroups)),
                       dim3(static_cast<unsigned>(waves * kWave)), 0, static_cast<hipStream_t>(stream), p);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return set_error(TD_E_LAUNCH, "probe_gather: %s", hipGetErrorString(e));
    return 0;
}
