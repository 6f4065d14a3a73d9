// Measured ceilings of the device: a read-only HBM stream and a dense MFMA
// loop.  Neither has a counterpart in the reference (it publishes no kernel
// figures); they give the benchmark a denominator measured on the same chip,
// beside the published peaks.
#include "vmi_device.h"
#include "vmi_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 8;  // 16-byte loads in flight per lane
constexpr size_t kChunk = (size_t)kThreads * kUnroll;  // 16-byte units per workgroup pass

// Workgroup b reads 32 KB chunks b, b + G, b + 2G, ... (G = gridDim.x); in a
// chunk, load u of lane t reads unit u * 256 + t, so every wave load is 1 KB
// of contiguous memory.  Nontemporal loads mark the lines for early eviction,
// as the MoE kernels' weight streams do.  Every 32-bit word is XORed into one
// value per workgroup, stored to sink[blockIdx.x] (a plain store: atomics on
// one shared word would serialise at the L2 and cost microseconds per launch).
template <bool NT>
__global__ __launch_bounds__(kThreads) void k_stream_read(const vmi_u4* __restrict__ src, size_t n16,
                                                          uint32_t* __restrict__ sink) {
    const size_t full = n16 / kChunk;
    vmi_u4 acc = {0u, 0u, 0u, 0u};
    const uint32_t voff = 16u * threadIdx.x;
    for (size_t c = blockIdx.x; c < full; c += gridDim.x) {
        // one buffer resource per chunk: the loads carry the cache policy
        const __amdgpu_buffer_rsrc_t r = vmi_rsrc(src + c * kChunk, (uint32_t)(16 * kChunk));
        vmi_u4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
            v[u] = NT ? vmi_bload_b128_nt(r, voff, 16u * kThreads * u) : vmi_bload_b128(r, voff, 16u * kThreads * u);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u];
    }
    // the tail (n16 not a multiple of the chunk): workgroup 0 alone
    if (blockIdx.x == 0)
        for (size_t i = full * kChunk + threadIdx.x; i < n16; i += kThreads) acc ^= src[i];
    __shared__ uint32_t s_x[kThreads / VMI_WAVE];
    uint32_t x = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if ((threadIdx.x & (VMI_WAVE - 1)) == 0) s_x[threadIdx.x / VMI_WAVE] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t w = 0;
#pragma unroll
        for (int i = 0; i < kThreads / VMI_WAVE; ++i) w ^= s_x[i];
        sink[blockIdx.x] = w;
    }
}

// Four independent accumulation chains per wave keep the matrix core busy
// while each MFMA's result is pending.  The operands are small exact fp16
// values, so the sums stay finite for any iteration count used here.
__global__ __launch_bounds__(kThreads) void k_mfma_peak(int iters, float* __restrict__ sink) {
    const int lane = threadIdx.x & (VMI_WAVE - 1);
    vmi_half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)((float)((lane + i) & 7) * 0.0009765625f);
        b[i] = (_Float16)((float)((lane * 3 + i) & 7) * 0.0009765625f);
    }
    vmi_f4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0;
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_16x16x32_f16(b, b, c3, 0, 0, 0);
    }
    const float s = (c0[0] + c1[1]) + (c2[2] + c3[3]);
    // lane 0 of each workgroup's first wave writes its sum: one store per
    // workgroup, into sink[blockIdx.x]
    if (threadIdx.x == 0) sink[blockIdx.x] = s;
}

}  // namespace

extern "C" int vmi_stream_read(const void* src, size_t bytes, int nontemporal, int workgroups, uint32_t* sink,
                               void* stream) {
    vmi::clear_error();
    if (!src || !sink) return vmi::fail(VMI_ERR_INVALID, "vmi_stream_read: null pointer");
    if (bytes == 0 || bytes % 16 || ((uintptr_t)src & 15))
        return vmi::fail(VMI_ERR_INVALID, "vmi_stream_read: bytes=%zu must be a non-zero multiple of 16 and src "
                                          "16-byte aligned", bytes);
    if (workgroups <= 0 || workgroups > 65536)
        return vmi::fail(VMI_ERR_INVALID, "vmi_stream_read: workgroups=%d outside [1, 65536]", workgroups);
    hipStream_t s = (hipStream_t)stream;
    const size_t n16 = bytes / 16;
    if (nontemporal)
        hipLaunchKernelGGL(k_stream_read<true>, dim3(workgroups), dim3(kThreads), 0, s, (const vmi_u4*)src, n16, sink);
    else
        hipLaunchKernelGGL(k_stream_read<false>, dim3(workgroups), dim3(kThreads), 0, s, (const vmi_u4*)src, n16,
                           sink);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_stream_read launch");
}

extern "C" int vmi_mfma_peak(int workgroups, int iters, float* sink, void* stream) {
    vmi::clear_error();
    if (!sink) return vmi::fail(VMI_ERR_INVALID, "vmi_mfma_peak: null sink");
    if (workgroups <= 0 || workgroups > 65536 || iters <= 0 || iters > (1 << 24))
        return vmi::fail(VMI_ERR_INVALID, "vmi_mfma_peak: workgroups=%d iters=%d out of range", workgroups, iters);
    hipLaunchKernelGGL(k_mfma_peak, dim3(workgroups), dim3(kThreads), 0, (hipStream_t)stream, iters, sink);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_mfma_peak launch");
}
