// Host-side internals shared by the libvmi translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/vmi.h"

namespace vmi {

// Records the thread-local error message and returns `code`.
int fail(int code, const char* fmt, ...);
int hip_fail(hipError_t e, const char* what);
void clear_error();

inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
int device_cus();  // compute units of the current device

constexpr int kRouteMaxPairs = 160;
constexpr int kRouteMaxT = 16;

// Routing of one verify batch as the down/combine kernel reads it, written by
// one workgroup of the gate/up kernel.
struct RouteInfo {
    int32_t U;                               // distinct valid slots
    int32_t uslot[kRouteMaxPairs];           // slot of distinct index u (first-appearance order)
    float wt[kRouteMaxPairs][kRouteMaxT];    // combine weight of (u, token): sum of its pairs' scores
    int32_t jr[kRouteMaxPairs][kRouteMaxT];  // rank j of the token's first pair on u, -1 if none: the
                                             // token's experts are added in rank order
    int32_t pv[kRouteMaxPairs];              // 1: pair p is its token's first pair on a valid slot
};

// Workspace carve-up of vmi_moe_layer (and its no-allocation variant).
struct MoeWorkspace {
    uint32_t* status;     // device status word (VMI_STATUS_*)
    RouteInfo* route;
    float* logits;        // [T, E]
    float* sg_logit;      // [T]
    uint32_t __attribute__((ext_vector_type(4)))* xop;    // [T, H/8] MFMA operands of the MoE input
    float* xsum;          // [T, H/64] per-group sums of those operands
    float* fscale;        // [T] power-of-two range factor of the operands
    uint16_t* part;       // [T*k + T, I/64, H] weighted bf16 partial rows: pair p's (or the shared
                          // expert's for token t, row T*k + t) down projection of each slice
    size_t bytes;
};

MoeWorkspace carve_workspace(void* base, int T, int k, int hidden, int inter, int num_experts);

// Quantised GEMV over up to three stacked matrices (k_qgemv, vmi_attn.hip):
// out[t][n] = sum_k x[t][k] W[n][k] for T <= 8 tokens, T * K <= 32768.
struct QgemvCall {
    const uint16_t* x;      // [T, K] bf16
    int T, K, bits;
    vmi_qmat m[3];
    int rows[3];            // rows of each matrix
    int nrows;              // total
    float* out;             // [T, out_stride] f32: row n of the stack at column n
    int out_stride;
    const uint16_t* residual;  // optional [T, out_stride] bf16: out_bf16 = bf16(y + residual)
    uint16_t* out_bf16;        // optional
    const uint16_t* norm_w;    // optional [K] bf16: x is first RMS-normalised (canonical order)
    float eps;
};
hipError_t launch_qgemv(const QgemvCall& q, hipStream_t s);
// Whether launch_qgemv can normalise x itself (QgemvCall::norm_w): the MFMA
// kernel with K in {512, 1024, 2048}.
bool qgemv_fuses_norm(const QgemvCall& q);
// bf16 RMSNorm of T rows of width H (H % 512 == 0) into out (stride H).
hipError_t launch_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int T, int H, uint16_t* out, hipStream_t s);
// Non-null, 16-byte aligned packed weights.
bool qmat_ok(const vmi_qmat& m);

}  // namespace vmi
