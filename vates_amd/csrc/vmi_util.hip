// Error reporting, dequantisation and synthetic-data kernels of libvmi.
#include <stdarg.h>
#include <stdio.h>

#include "vmi_device.h"
#include <atomic>

#include "vmi_internal.h"

namespace {
thread_local char g_err[512] = {0};
constexpr int kThreads = 256;
}  // namespace

namespace vmi {

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(VMI_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

void clear_error() { g_err[0] = 0; }

// Compute units of the current device, queried once per device.  The cache
// entries are atomics: threads calling at once may each query, and all store
// the same value, so the function is re-entrant without a lock.
int device_cus() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    const int known = cached[dev].load(std::memory_order_relaxed);
    if (known > 0) return known;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

}  // namespace vmi

extern "C" const char* vmi_last_error(void) { return g_err; }
extern "C" int vmi_version(void) { return 1; }

// ------------------------------------------------------------------ dequant
namespace {

__global__ void k_dequant(vmi_qmat m, int rows, int cols, int group, int bits, float* out) {
    const int64_t n = (int64_t)rows * cols;
    const int words = cols * bits / 32, groups = cols / group;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / cols;
        const int c = (int)(i - r * cols);
        const int bit = c * bits;
        const uint32_t q = (m.w[r * words + bit / 32] >> (bit % 32)) & ((1u << bits) - 1u);
        const int64_t sb = r * groups + c / group;
        out[i] = fmaf((float)q, vmi_bf16_to_f32(m.s[sb]), vmi_bf16_to_f32(m.b[sb]));
    }
}

// Philox4x32-10 (Salmon et al., SC'11).
__device__ __forceinline__ void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
        const uint32_t n0 = hi1 ^ c[1] ^ k0;
        const uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

// Two synthetic values (elements 2*pair and 2*pair+1) of one stream.
__device__ __forceinline__ void synth_pair(uint64_t seed, uint32_t stream, uint64_t pair, float scale, float& v0,
                                           float& v1) {
    uint32_t c[4] = {(uint32_t)pair, (uint32_t)(pair >> 32), stream, 0x5eed0001u};
    philox(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    const int32_t s0 = (int32_t)((c[0] & 0xffffu) + (c[0] >> 16) + (c[1] & 0xffffu) + (c[1] >> 16)) - 131070;
    const int32_t s1 = (int32_t)((c[2] & 0xffffu) + (c[2] >> 16) + (c[3] & 0xffffu) + (c[3] >> 16)) - 131070;
    v0 = (float)s0 * scale;
    v1 = (float)s1 * scale;
}

// One thread per (row, group of 64): draw, min/max, bf16 scale/bias, quantise.
template <int BITS>
__global__ void k_synth_quant(uint64_t seed, uint32_t stream, int64_t rows, int cols, float scale, uint32_t* w,
                              uint16_t* s, uint16_t* b) {
    constexpr int kGroup = 64;
    constexpr int kQmax = (1 << BITS) - 1;
    constexpr int kWords = kGroup * BITS / 32;
    const int groups = cols / kGroup;
    const int64_t ng = rows * groups;
    for (int64_t gi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; gi < ng; gi += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = gi / groups;
        const int g = (int)(gi - r * groups);
        const uint64_t e0 = (uint64_t)r * cols + (uint64_t)g * kGroup;  // even: cols and 64 are even
        float v[kGroup];
#pragma unroll
        for (int i = 0; i < kGroup; i += 2) synth_pair(seed, stream, (e0 + i) >> 1, scale, v[i], v[i + 1]);
        float mn = v[0], mx = v[0];
#pragma unroll
        for (int i = 1; i < kGroup; ++i) {
            if (v[i] < mn) mn = v[i];
            if (v[i] > mx) mx = v[i];
        }
        float sc = (mx - mn) / (float)kQmax;
        if (sc == 0.0f) sc = 1.0f;
        uint16_t sb = vmi_f32_to_bf16(sc);
        const uint16_t bb = vmi_f32_to_bf16(mn);
        float sf = vmi_bf16_to_f32(sb);
        const float bf = vmi_bf16_to_f32(bb);
        if (sf == 0.0f) {
            sb = 0x3f80;
            sf = 1.0f;
        }
        uint32_t words[kWords];
#pragma unroll
        for (int i = 0; i < kWords; ++i) words[i] = 0u;
#pragma unroll
        for (int i = 0; i < kGroup; ++i) {
            const float qf = roundf(__fdiv_rn(v[i] - bf, sf));
            int q = (int)qf;
            if (!(qf >= 0.0f)) q = 0;
            if (q > kQmax) q = kQmax;
            words[(i * BITS) / 32] |= ((uint32_t)q) << ((i * BITS) % 32);
        }
        uint32_t* wo = w + (r * cols + (int64_t)g * kGroup) * BITS / 32;
#pragma unroll
        for (int i = 0; i < kWords; ++i) wo[i] = words[i];
        s[gi] = sb;
        b[gi] = bb;
    }
}

__global__ void k_synth_bf16(uint64_t seed, uint32_t stream, int64_t n, float scale, uint16_t* out) {
    const int64_t npair = (n + 1) / 2;
    for (int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; p < npair; p += (int64_t)gridDim.x * blockDim.x) {
        float v0, v1;
        synth_pair(seed, stream, (uint64_t)p, scale, v0, v1);
        out[2 * p] = vmi_f32_to_bf16(v0);
        if (2 * p + 1 < n) out[2 * p + 1] = vmi_f32_to_bf16(v1);
    }
}

int grid_for(int64_t n) {
    const int64_t g = (n + kThreads - 1) / kThreads;
    return (int)(g < 65536 ? (g > 0 ? g : 1) : 65536);
}

}  // namespace

extern "C" int vmi_dequant_affine(vmi_qmat m, int rows, int cols, int group, int bits, float* out, void* stream) {
    vmi::clear_error();
    if (!m.w || !m.s || !m.b || !out) return vmi::fail(VMI_ERR_INVALID, "null pointer");
    if (rows <= 0 || cols <= 0 || group <= 0 || cols % group || (bits != 4 && bits != 8) || (cols * bits) % 32)
        return vmi::fail(VMI_ERR_INVALID, "bad shape rows=%d cols=%d group=%d bits=%d", rows, cols, group, bits);
    hipLaunchKernelGGL(k_dequant, dim3(grid_for((int64_t)rows * cols)), dim3(kThreads), 0,
                       static_cast<hipStream_t>(stream), m, rows, cols, group, bits, out);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_dequant launch");
}

extern "C" int vmi_synth_quantized(uint64_t seed, uint32_t stream_id, int64_t rows, int cols, int group, int bits,
                                   float scale, uint32_t* w, uint16_t* s, uint16_t* b, void* stream) {
    vmi::clear_error();
    if (!w || !s || !b) return vmi::fail(VMI_ERR_INVALID, "null pointer");
    if (rows <= 0 || cols <= 0 || cols % 64) return vmi::fail(VMI_ERR_INVALID, "bad shape rows=%lld cols=%d",
                                                              (long long)rows, cols);
    if (group != 64 || (bits != 4 && bits != 8))
        return vmi::fail(VMI_ERR_UNSUPPORTED, "synthetic quantiser built for group=64, bits 4/8");
    const int64_t ng = rows * (cols / 64);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    if (bits == 4)
        hipLaunchKernelGGL(k_synth_quant<4>, dim3(grid_for(ng)), dim3(kThreads), 0, st, seed, stream_id, rows, cols,
                           scale, w, s, b);
    else
        hipLaunchKernelGGL(k_synth_quant<8>, dim3(grid_for(ng)), dim3(kThreads), 0, st, seed, stream_id, rows, cols,
                           scale, w, s, b);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_synth_quant launch");
}

extern "C" int vmi_synth_bf16(uint64_t seed, uint32_t stream_id, int64_t n, float scale, uint16_t* out,
                              void* stream) {
    vmi::clear_error();
    if (!out || n <= 0) return vmi::fail(VMI_ERR_INVALID, "null output or n<=0");
    hipLaunchKernelGGL(k_synth_bf16, dim3(grid_for((n + 1) / 2)), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                       seed, stream_id, n, scale, out);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_synth_bf16 launch");
}
