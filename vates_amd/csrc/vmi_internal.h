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

constexpr int kRouteMaxPairs = 160;
constexpr int kRouteMaxT = 16;

// Routing of one verify batch as the down/combine kernel reads it, written by
// one workgroup of the gate/up kernel.
struct RouteInfo {
    int32_t U;                               // distinct valid slots
    int32_t uslot[kRouteMaxPairs];           // slot of distinct index u (first-appearance order)
    float wt[kRouteMaxPairs][kRouteMaxT];    // combine weight of (u, token): sum of its pairs' scores
};

// Workspace carve-up shared by vmi_fused_moe_slots and vmi_moe_layer.  Expert
// activations are indexed by distinct slot u < T*k; index T*k is the shared
// expert.
struct MoeWorkspace {
    uint32_t* status;     // device status word (VMI_STATUS_*)
    RouteInfo* route;
    float* logits;        // [T, E]
    float* sg_logit;      // [T]
    uint32_t __attribute__((ext_vector_type(4)))* xop;    // [T, H/8] MFMA operands of the MoE input
    float* xsum;          // [T, H/64] per-group sums of those operands
    float* fscale;        // [T] power-of-two range factor of the operands
    uint32_t __attribute__((ext_vector_type(4)))* actop;  // [T*k+1, T, I/8] bf16 down-projection operands
    float* axs;           // [T*k+1, T, I/64] per-group activation sums
    size_t bytes;
};

MoeWorkspace carve_workspace(void* base, int T, int k, int hidden, int inter, int num_experts);

}  // namespace vmi
