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

// Distinct-slot table of one verify batch, written by one workgroup.
struct RouteInfo {
    int32_t U;                                  // distinct valid slots
    int32_t uslot[kRouteMaxPairs];              // slot of distinct index u
    uint32_t umask[kRouteMaxPairs];             // tokens routed to u
    int16_t upair[kRouteMaxPairs][kRouteMaxT];  // first pair (t*k+j) of (u, t), -1 if none
    int32_t psrc[kRouteMaxPairs];               // pair whose partial output serves pair p, -1 if invalid
};

// Workspace carve-up shared by vmi_fused_moe_slots and vmi_moe_layer.
struct MoeWorkspace {
    uint32_t* status;     // device status word (VMI_STATUS_*)
    RouteInfo* route;
    float* logits;        // [T, E]
    float* sg_logit;      // [T]
    float* sg;            // [T]
    int32_t* ids;         // [T*k]
    float* scores;        // [T*k]
    int32_t* slots;       // [T*k]
    uint32_t __attribute__((ext_vector_type(4)))* xop;  // [T, H/64, 4, 2] MFMA operands
    float* xsum;          // [T, H/64]
    float* fscale;        // [T]
    float* part;          // [T*k + T, inter/64, hidden] per-slice partial outputs
    size_t bytes;
};

MoeWorkspace carve_workspace(void* base, int T, int k, int hidden, int inter, int num_experts);

}  // namespace vmi
