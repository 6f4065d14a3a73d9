// Fused 4-bit MoE for the speculative-decode verify batch (T <= 16 tokens).
//
// Three stream-ordered kernels per layer; kernel boundaries carry every
// cross-workgroup dependency (no fences, no counters, no spin waits):
//   k_router    router logits, one wave per (router row, token): each wave
//               normalises its token's input itself (the optional pre-MoE
//               RMSNorm) and accumulates the logit in a fixed fp32 order
//               (bit-identical to the CPU oracle).  One spare wave per token
//               writes the MoE input in MFMA operand order.
//   k_gateup    one workgroup per (distinct slot, 64-row slice of the
//               intermediate dimension), shared-expert slices first.  Every
//               workgroup first routes the batch itself from the logits
//               (softmax, top-k, renorm, slot table, distinct slots) - the
//               same deterministic result in every workgroup - so no routing
//               kernel sits between router and experts.  Wave w owns rows
//               16w..16w+15 of the slice in gate and in up over the whole
//               hidden dimension; SwiGLU happens in registers and the slice's
//               64 activations are written as down-projection MFMA operands
//               (one quantisation group of down).
//   k_down_rows one workgroup per 8 output rows: every distinct slot's down
//               projection for those rows, the combine weights, the gated
//               shared expert and the residual, summed in a fixed order.
// vmi_fused_moe_slots runs k_prep (operands only) in place of k_router and
// routes from the caller's slot list inside k_gateup.
//
// 4-bit weights enter v_mfma_f32_16x16x32_f16 as exact fp16 subnormals.  One
// 16-byte load per lane covers 16 rows x 64 bytes = two quantisation groups;
// for T <= 8 both groups share one MFMA: tokens of the even group occupy A
// rows 0..7 (K blocks 0-1), tokens of the odd group rows 8..15 (K blocks 2-3).
//
// Semantics follow native/ext/compute/fused_moe.cpp:221-298 (slot pair kernel
// and reduce_pairs) and mlx_streaming/core/moe/block.py:102-109, 321-329, 1008.

#include <mutex>

#include "vmi_device.h"
#include "vmi_internal.h"

VMI_TL_DECL

namespace {

constexpr int kThreads = 256;
constexpr int kMaxT = 16;
constexpr int kMaxPairs = 160;
constexpr int kMaxK = 16;
constexpr int kMaxE = 1024;
constexpr int kSlice = 64;        // intermediate rows per k_gateup workgroup (= one down group)
constexpr int kMaxInter = 512;
constexpr int kFirstTable = 1024; // LDS first-occurrence table covers cap <= 1024
constexpr float kTwo24 = 16777216.0f;

static_assert(kMaxPairs == vmi::kRouteMaxPairs && kMaxT == vmi::kRouteMaxT, "route table sizes");

using vmi::RouteInfo;

// Wave index within the workgroup as a scalar (uniform) value, so values and
// buffer descriptors derived from it stay in SGPRs.
__device__ __forceinline__ int vmi_wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }
__device__ __forceinline__ int vmi_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ float vmi_bf16r(float v) { return vmi_bf16_to_f32(vmi_f32_to_bf16(v)); }

__device__ __forceinline__ void unpack_bf16x8(const uint4& q, float (&v)[8]) {
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(qw[i] << 16);
        v[2 * i + 1] = __uint_as_float(qw[i] & 0xffff0000u);
    }
}

// ------------------------------------------------------------ operands
// f16 activation operand for one packed word's 8 columns: slot s holds column
// perm[s] = {0,4,1,5,2,6,3,7}[s], divided by 16 for s in {2,3,6,7} (see
// vmi_unpack_u4_f16); xsum accumulates the values the MFMA effectively
// multiplies (x'' per column), used by the affine-bias term.
__device__ __forceinline__ vmi_u4 make_act_operand(const float (&xv)[8], float f, float& xsum) {
    const _Float16 h0 = (_Float16)(xv[0] * f), h1 = (_Float16)(xv[4] * f);
    const _Float16 h2 = (_Float16)(xv[1] * f * 0.0625f), h3 = (_Float16)(xv[5] * f * 0.0625f);
    const _Float16 h4 = (_Float16)(xv[2] * f), h5 = (_Float16)(xv[6] * f);
    const _Float16 h6 = (_Float16)(xv[3] * f * 0.0625f), h7 = (_Float16)(xv[7] * f * 0.0625f);
    xsum += (float)h0 + (float)h1 + (float)h4 + (float)h5 +
            16.0f * ((float)h2 + (float)h3 + (float)h6 + (float)h7);
    vmi_u4 r;
    r[0] = vmi_h2_bits(h0, h1);
    r[1] = vmi_h2_bits(h2, h3);
    r[2] = vmi_h2_bits(h4, h5);
    r[3] = vmi_h2_bits(h6, h7);
    return r;
}

// Canonical inverse rms shared with the CPU oracle: lane l of a wave holds
// columns [l*cpl, (l+1)*cpl) (cpl/8 packed chunks); x^2 summed with fmaf in
// column order, the canonical wave-sum tree, then 1/sqrt(ss/H + eps) with
// correctly rounded sqrt and division.  Every lane returns the same value.
template <int NCH>
__device__ __forceinline__ float canonical_inv_rms(const uint4 (&xr)[NCH], int H, float eps) {
    float ss = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        float v[8];
        unpack_bf16x8(xr[ch], v);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(v[i], v[i], ss);
    }
    ss = vmi_wave_sum_canon(ss);
    return __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / (float)H) + eps));
}

struct OperandOut {
    vmi_u4* xop;    // [T, H/8] MFMA operands
    float* xsum;    // [T, H/64]
    float* fscale;  // [T]
};

// ---------------------------------------------------------------- router
struct RouterArgs {
    const uint16_t* x;
    const uint16_t* norm_w;
    float eps;
    int T, H, E;
    vmi_qmat router;
    int rbits;
    const float* bias;
    vmi_qmat sgate;
    int sgbits, has_sgate;
    int row_wgs;      // row groups (four waves of kRouterRows rows each) per token
    float* logits;    // [T, E]
    float* sg_logit;  // [T]
    OperandOut ops;
};

// MFMA operands of token t written by one wave from its (normalised) input in
// registers: lane l holds packed chunks xr[ch] = columns 8(l*NCH + ch) ..
// +7.  The same values, range factor and group sums as write_operands: each
// 64-column group's sum runs the butterfly over its 8 chunk sums (strides 1,
// 2, 4 chunks; within the lane where the stride is below NCH, across lanes
// above), the same additions up to operand order.
template <int NCH>
__device__ __forceinline__ void operands_from_wave(const uint4 (&xr)[NCH], int H, int t, const OperandOut& o) {
    const int lane = threadIdx.x & 63;
    float v[NCH][8];
    float amax = 0.0f;
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        unpack_bf16x8(xr[ch], v[ch]);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[ch][i]));
    }
    amax = vmi_wave_max(amax);
    const float f = vmi_fp16_range_scale(amax);
    float xs[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        xs[ch] = 0.0f;
        o.xop[(size_t)t * (H / 8) + lane * NCH + ch] = make_act_operand(v[ch], f, xs[ch]);
    }
#pragma unroll
    for (int st = 1; st < 8; st *= 2) {
        if (st < NCH) {
            float nx[NCH];
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) nx[ch] = xs[ch] + xs[ch ^ st];
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) xs[ch] = nx[ch];
        } else {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) xs[ch] += __shfl_xor(xs[ch], st / NCH, VMI_WAVE);
        }
    }
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const int k = lane * NCH + ch;
        if ((k & 7) == 0) o.xsum[(size_t)t * (H / 64) + k / 8] = xs[ch];
    }
    if (lane == 0) o.fscale[t] = f;
}

// Router rows for one token per workgroup: workgroup i covers row group b
// (wave w takes rows RW (4b + w) .. + RW - 1) for token t, where the T
// workgroups of a row group sit on one XCD (workgroups are dealt to the 8
// XCDs round-robin by index), so the rows' weights reach that XCD's L2 once.
// Row E is the shared-expert gate; the wave whose first row is the first
// multiple of RW at or past E + has_sgate (the row groups always cover it)
// writes token t's MFMA operands instead of logits.
// Each wave loads token t's input with lane l owning columns
// [l*CPL, (l+1)*CPL): the canonical inverse rms, the bf16-rounded normalised
// input (once for its RW rows), then per row fmaf(w, x, acc) in column
// order; the 64 partials meet in the canonical wave-sum tree.  No LDS and no
// barrier: a wave depends on nothing but its own loads.  The CPU oracle
// reproduces this order bit for bit (orc_router_logits_f32).
constexpr int kRouterRows = 2;  // router rows per wave

template <int CPL>
__global__ __launch_bounds__(kThreads) void k_router(RouterArgs a) {
    constexpr int NCH = CPL / 8;  // packed 8-column chunks per lane
    constexpr int RW = kRouterRows;
    VMI_STAMP(0, 0);
    // every argument in SGPRs at once: one scalar round trip for the argument
    // block, not one per field as the code first needs it
    asm volatile("" ::"s"(a.x), "s"(a.norm_w), "s"(a.eps), "s"(a.T), "s"(a.H), "s"(a.E), "s"(a.router.w),
                 "s"(a.router.s), "s"(a.router.b), "s"(a.rbits), "s"(a.bias));
    asm volatile("" ::"s"(a.sgate.w), "s"(a.sgate.s), "s"(a.sgate.b), "s"(a.sgbits), "s"(a.has_sgate),
                 "s"(a.row_wgs), "s"(a.logits), "s"(a.sg_logit), "s"(a.ops.xop), "s"(a.ops.xsum), "s"(a.ops.fscale));
    const int lane = threadIdx.x & 63, w = vmi_wave_id();
    const int T = a.T, H = a.H;
    const int G = H / 64;
    const int xcd = (int)blockIdx.x & 7, jb = (int)blockIdx.x >> 3;
    const int t = jb % T, b = (jb / T) * 8 + xcd;
    if (b >= a.row_wgs) return;
    const int c0 = lane * CPL;
    const int row0 = RW * (b * (kThreads / VMI_WAVE) + w);
    const int nrows = a.E + a.has_sgate;
    const int ops_row = RW * ((nrows + RW - 1) / RW);
    const bool is_ops = row0 == ops_row;
    if (row0 >= nrows && !is_ops) return;
    // the input and the norm weights first (the normalisation needs them),
    // then the router rows; loads retire in issue order
    const __amdgpu_buffer_rsrc_t rx = vmi_rsrc(a.x + (size_t)t * H, (uint32_t)H * 2u);
    const __amdgpu_buffer_rsrc_t rn = vmi_rsrc(a.norm_w ? a.norm_w : a.x, a.norm_w ? (uint32_t)H * 2u : 0u);
    uint4 xr[NCH], nwv[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const vmi_u4 xv = vmi_bload_b128(rx, (uint32_t)(c0 + 8 * ch) * 2u, 0);
        const vmi_u4 nv = vmi_bload_b128(rn, (uint32_t)(c0 + 8 * ch) * 2u, 0);
        xr[ch] = make_uint4(xv[0], xv[1], xv[2], xv[3]);
        nwv[ch] = make_uint4(nv[0], nv[1], nv[2], nv[3]);
    }
    asm volatile("" ::: "memory");
    // each row's words (8-bit: CPL/4 words of this lane's columns, 4-bit:
    // CPL/8), its scale and bias, and its logit bias, by the same loads for
    // either width (an 8-bit share is CPL/16 16-byte pieces; a 4-bit share
    // uses the first CPL/32 of them, the rest reads past it unused; single
    // words where 16-byte pieces would not stay aligned): no branch, so no
    // wait for loads in flight ahead of them
    uint32_t wword[RW][CPL / 4], sv[RW], bv[RW];
    float rbias[RW];
    bool row_ok[RW], is_sg[RW];
    int bitsr[RW];
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        const int row = row0 + j;
        row_ok[j] = row < nrows;
        is_sg[j] = row_ok[j] && row >= a.E;  // wave-uniform
        const vmi_qmat m = is_sg[j] ? a.sgate : a.router;
        const int bits = is_sg[j] ? a.sgbits : a.rbits;
        bitsr[j] = bits;
        const int r = is_sg[j] ? 0 : (row_ok[j] ? row : 0);
        const uint32_t row_words = (uint32_t)(H * bits / 32);
        const __amdgpu_buffer_rsrc_t rw = vmi_rsrc(m.w + (size_t)r * row_words, row_ok[j] ? row_words * 4u : 0u);
        const __amdgpu_buffer_rsrc_t rs = vmi_rsrc(m.s + (size_t)r * G, row_ok[j] ? (uint32_t)G * 2u : 0u);
        const __amdgpu_buffer_rsrc_t rb = vmi_rsrc(m.b + (size_t)r * G, row_ok[j] ? (uint32_t)G * 2u : 0u);
        const uint32_t wbase = (uint32_t)(c0 * bits / 32) * 4u;
        if constexpr (CPL >= 32) {
            vmi_u4 wq[CPL / 16];
#pragma unroll
            for (int i = 0; i < CPL / 16; ++i) wq[i] = vmi_bload_b128_nt(rw, wbase + 16u * i, 0);
#pragma unroll
            for (int i = 0; i < CPL / 4; ++i) wword[j][i] = wq[i / 4][i % 4];
        } else {
#pragma unroll
            for (int i = 0; i < CPL / 4; ++i) wword[j][i] = vmi_bload_b32_nt(rw, wbase + 4u * i, 0);
        }
        sv[j] = vmi_bload_b16(rs, (uint32_t)(c0 / 64) * 2u, 0);
        bv[j] = vmi_bload_b16(rb, (uint32_t)(c0 / 64) * 2u, 0);
        const bool has_bias = a.bias != nullptr && row_ok[j] && !is_sg[j];
        rbias[j] = __uint_as_float(vmi_bload_b32(
            vmi_rsrc(has_bias ? a.bias : a.logits, has_bias ? 4u * (uint32_t)a.E : 0u), 4u * (uint32_t)r, 0));
    }
    VMI_STAMP(0, 2);
    if (a.norm_w) {
        const float inv = canonical_inv_rms<NCH>(xr, H, a.eps);
        VMI_STAMP(0, 3);
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            float xf[8], nw[8];
            unpack_bf16x8(xr[ch], xf);
            unpack_bf16x8(nwv[ch], nw);
            uint32_t pk[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                pk[i] = vmi_pack_bf16x2((xf[2 * i] * inv) * nw[2 * i], (xf[2 * i + 1] * inv) * nw[2 * i + 1]);
            xr[ch] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        }
    }
    if (is_ops) {
        operands_from_wave<NCH>(xr, H, t, a.ops);
        VMI_STAMP_WAVE(0, 8);
        return;
    }
    VMI_STAMP(0, 4);
#pragma unroll
    for (int j = 0; j < RW; ++j) {
        if (!row_ok[j]) continue;  // wave-uniform
        // dequantised weights (w = q*s + b is exact in fp32), one fmaf chain in column order
        const float sc = vmi_bf16_to_f32(sv[j]), bi = vmi_bf16_to_f32(bv[j]);
        const int bits = bitsr[j];
        float acc = 0.0f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            float xf[8];
            unpack_bf16x8(xr[ch], xf);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int c = 8 * ch + i;
                const uint32_t qv = (bits == 4) ? (wword[j][c / 8] >> (4 * (c % 8))) & 15u
                                                : (wword[j][c / 4] >> (8 * (c % 4))) & 255u;
                acc = fmaf(fmaf((float)qv, sc, bi), xf[i], acc);
            }
        }
        const float v = vmi_wave_sum_canon(acc);
        if (lane == 0) {
            if (is_sg[j]) {
                a.sg_logit[t] = v;
            } else {
                float lv = v;
                if (a.bias != nullptr) lv = lv + rbias[j];
                a.logits[(size_t)t * a.E + row0 + j] = lv;
            }
        }
    }
    VMI_STAMP(0, 1);
    VMI_STAMP_WAVE(0, 8);
}

// ----------------------------------------------------------- routing
// Routing state of one verify batch while it is being built, in LDS.
struct RouteLds {
    int32_t ids[kMaxPairs];
    float scores[kMaxPairs];
    int32_t slot[kMaxPairs];   // -1 = invalid
    int32_t rank[kMaxPairs];   // distinct index, stored at first-occurrence pairs
    int32_t uslot[kMaxPairs];
    uint32_t umask[kMaxPairs];
    int32_t wcnt[kThreads / VMI_WAVE];
    int32_t U;
    uint32_t bad;
};

// Top-k rank key of logit l at expert index e: order key of the value in the
// high word (larger value first; -0 folded into +0; NaN maps to 1, below
// every number) and ~e in the low word (lower index first on ties).  Keys are
// unique, so a wave-wide maximum names one winner; 0 marks a taken slot.
__device__ __forceinline__ uint64_t topk_rank_key(float f, int e) {
    uint32_t u = __float_as_uint(f);
    u = (u == 0x80000000u) ? 0u : u;
    const uint32_t ok = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t hi = (f != f) ? 1u : ok;
    return ((uint64_t)hi << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}


// Softmax + top-k + renorm of token t's logits by one wave (block.py:321-329).
// Lane l holds experts l + 64i (i < NI) as rank keys, sorted descending once
// (bitonic network); each of the k rounds (a rolled loop: this code runs once
// per workgroup, so it is kept small for the instruction cache) takes the
// wave-wide maximum of the lanes' heads and the winning lane records and pops
// its head.  Lane j then reads the j-th selection; exp, the renormalising sum
// (in j order) and the scores are lane-parallel.
template <int NI>
__device__ void topk_token(const float (&v)[NI], int E, int k, int norm, int t, RouteLds& R) {
    const int lane = threadIdx.x & 63;
    const int nreal = E >> 6;  // E is a multiple of 64: slot i is real for i < E/64 (uniform)
    uint64_t key[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const uint64_t kk = topk_rank_key(v[i], lane + 64 * i);
        key[i] = (i < nreal) ? kk : 0ull;
    }
    asm volatile("" ::"v"(key[NI - 1]));
    VMI_STAMP(1, 9);
#pragma unroll
    for (int size = 2; size <= NI; size *= 2)
#pragma unroll
        for (int stride = size / 2; stride > 0; stride /= 2)
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int j = i ^ stride;
                if (j > i) vmi_cx64(key[i], key[j], (i & size) == 0);
            }
    // each round: the wave maximum of the 32-bit value keys of the lane heads;
    // the lane holding it (a ballot names it; equal values fall back to the
    // full (value, index) key) writes its expert and value into the round's
    // entry itself, so no key is broadcast
    // round j's winner goes to lane j's registers (its index word and value
    // key read from the winning lane), so the loop has no LDS traffic
    uint32_t my_lo = 0u, my_hv = 0u;
#pragma unroll 1
    for (int j = 0; j < k; ++j) {
        const uint32_t hv = (uint32_t)(key[0] >> 32);
        const uint32_t Mv = vmi_wave_max_u32(hv);
        const uint64_t cand = __ballot(hv == Mv);
        uint64_t winm = cand;
        if (__popcll(cand) != 1) {
            const uint64_t M = vmi_wave_max_u64(hv == Mv ? key[0] : 0ull);
            winm = __ballot(key[0] == M);
        }
        const int wl = __builtin_ctzll(winm);  // uniform
        const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key[0], wl);
        my_lo = lane == j ? lo : my_lo;
        my_hv = lane == j ? Mv : my_hv;
        if (lane == wl) {
#pragma unroll
            for (int i = 0; i + 1 < NI; ++i) key[i] = key[i + 1];
            key[NI - 1] = 0ull;
        }
    }
    VMI_STAMP(1, 10);
    const int my_idx = lane < k ? (int)(0xffffffffu - my_lo) : 0;
    const float my_val = lane < k ? vmi_order_key_value(my_hv) : 0.0f;
    const float mx = vmi_readlane_f32(my_val, 0);
    const bool sel = lane < k;
    const bool bad = __ballot(sel && !(fabsf(my_val) < 3.0e38f)) != 0;
    const float e = sel ? expf(my_val - mx) : 0.0f;
    float den = 0.0f;
    if (norm) {
#pragma unroll 1
        for (int j = 0; j < k; ++j) den = den + vmi_readlane_f32(e, j);
    } else {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            if (i < nreal) part = part + expf(v[i] - mx);
        den = vmi_wave_sum_canon(part);
    }
    if (sel) {
        R.ids[t * k + lane] = my_idx;
        R.scores[t * k + lane] = e / den;
    }
    if (bad && lane == 0) atomicOr(&R.bad, VMI_STATUS_BAD_ROUTE);
}

template <int NI>
__device__ __forceinline__ void topk_load(const float* __restrict__ lt, int E, float (&v)[NI]) {
    const int lane = threadIdx.x & 63;
    const __amdgpu_buffer_rsrc_t rl = vmi_rsrc(lt, (uint32_t)E * 4u);
#pragma unroll
    for (int i = 0; i < NI; ++i) v[i] = __uint_as_float(vmi_bload_b32(rl, (uint32_t)(lane + 64 * i) * 4u, 0));
}

// Top-k of every token of the batch (wave w: tokens w, w + 4, ...), with the
// slot table staged alongside: the first token's logits and the table are
// loaded together, so their latencies overlap.
template <int NI>
__device__ void route_topk(const float* __restrict__ logits, int T, int E, int k, int norm, const int32_t* table,
                           int32_t* s_table, RouteLds& R) {
    const int tid = threadIdx.x, w = vmi_wave_id();
    float v[NI];
    if (w < T) topk_load<NI>(logits + (size_t)w * E, E, v);
    if (table) {
        const __amdgpu_buffer_rsrc_t rt = vmi_rsrc(table, (uint32_t)E * 4u);
        int32_t tv[kMaxE / kThreads];
#pragma unroll
        for (int i = 0; i < kMaxE / kThreads; ++i) tv[i] = (int32_t)vmi_bload_b32(rt, (uint32_t)(tid + kThreads * i) * 4u, 0);
#pragma unroll
        for (int i = 0; i < kMaxE / kThreads; ++i) s_table[tid + kThreads * i] = tv[i];
    }
    for (int t = w; t < T; t += kThreads / VMI_WAVE) {
        if (t != w) topk_load<NI>(logits + (size_t)t * E, E, v);
        topk_token<NI>(v, E, k, norm, t, R);
    }
}

__device__ void route_topk_dispatch(const float* __restrict__ logits, int T, int E, int k, int norm,
                                    const int32_t* table, int32_t* s_table, RouteLds& R) {
    if (E <= 64)
        route_topk<1>(logits, T, E, k, norm, table, s_table, R);
    else if (E <= 128)
        route_topk<2>(logits, T, E, k, norm, table, s_table, R);
    else if (E <= 256)
        route_topk<4>(logits, T, E, k, norm, table, s_table, R);
    else if (E <= 512)
        route_topk<8>(logits, T, E, k, norm, table, s_table, R);
    else
        route_topk<16>(logits, T, E, k, norm, table, s_table, R);
}

// Distinct valid slots in first-appearance order over the token-major pair
// list (R.slot filled, -1 = invalid).  cap <= kFirstTable uses an LDS
// first-occurrence table (only the entries of slots in use are touched).
// Fills rank/uslot/umask/U.  Called by all threads of a 256-thread workgroup.
__device__ void dedup_lds(int npairs, int k, int cap, RouteLds& R, int32_t* s_first) {
    const int tid = threadIdx.x, lane = tid & 63, w = vmi_wave_id();
    const bool table = cap <= kFirstTable;
    if (tid < kMaxPairs) R.umask[tid] = 0u;
    const int s = (tid < npairs) ? R.slot[tid] : -1;
    if (table && s >= 0) s_first[s] = 0x7fffffff;
    __syncthreads();
    if (table && s >= 0) atomicMin(&s_first[s], tid);
    __syncthreads();
    int fidx = -1;
    if (s >= 0) {
        if (table) {
            fidx = s_first[s];
        } else {
            fidx = tid;
            for (int q = 0; q < tid; ++q) {
                if (R.slot[q] == s) {
                    fidx = q;
                    break;
                }
            }
        }
    }
    const bool first = s >= 0 && fidx == tid;
    const uint64_t bal = __ballot(first);
    if (lane == 0) R.wcnt[w] = __popcll(bal);
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += R.wcnt[i];
    const int rank = base + __popcll(bal & ((1ull << lane) - 1ull));
    if (first) {
        R.rank[tid] = rank;
        R.uslot[rank] = s;
    }
    __syncthreads();
    if (s >= 0) atomicOr(&R.umask[R.rank[fidx]], 1u << (tid / k));
    if (tid == 0) {
        int U = 0;
        for (int i = 0; i < kThreads / VMI_WAVE; ++i) U += R.wcnt[i];
        R.U = U;
    }
    __syncthreads();
}

// ------------------------------------------------------------- experts
// Routing inputs and outputs shared by the two routed kernels (k_experts on
// the router's logits, k_gateup_f32 on a caller's slot list).
struct RouteArgs {
    int T, I, k, E, npairs;
    int from_slots;               // 1: caller slots + scores, 0: route from logits
    int norm, cap;
    const float* logits;          // [T, E]
    const int32_t* table;         // [E] or nullptr
    const int32_t* slots;         // [T*k] (from_slots), or nullptr: pair p uses matrix p
    const float* in_scores;       // [T*k] (from_slots)
    RouteInfo* route;             // written by the first routed workgroup
    uint32_t* status;
    int32_t* ids_out;             // [T*k] or nullptr
    float* scores_out;            // [T*k] or nullptr
};

// Slot table and first-appearance distinct slots of a batch of at most 64
// pairs by one wave (lane p: pair p), after the top-k: the same result as the
// workgroup-wide path below (a slot's distinct index is the number of
// distinct slots whose first pair comes earlier), with wave-level ordering of
// the LDS table instead of workgroup barriers.
__device__ void slots_dedup_wave(const RouteArgs& a, RouteLds& R, const int32_t* s_table, int32_t* s_first) {
    const int lane = threadIdx.x & 63;
    const int npairs = a.npairs, k = a.k;
    const bool pair = lane < npairs;
    int sl = -1;
    if (pair) {
        const int id = R.ids[lane];
        sl = (id >= 0 && id < a.E) ? (a.table ? s_table[id] : id) : -1;
        if (sl < 0 || sl >= a.cap) {
            sl = -1;
            atomicOr(&R.bad, VMI_STATUS_BAD_SLOT);
        }
        R.slot[lane] = sl;
        R.umask[lane] = 0u;
        if (sl >= 0) s_first[sl] = 0x7fffffff;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (sl >= 0) atomicMin(&s_first[sl], lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int fidx = sl >= 0 ? s_first[sl] : -1;
    const uint64_t bal = __ballot(sl >= 0 && fidx == lane);
    if (sl >= 0) {
        const int u = __popcll(bal & ((1ull << fidx) - 1ull));  // distinct index of the pair's slot
        if (fidx == lane) R.uslot[u] = sl;
        atomicOr(&R.umask[u], 1u << (lane / k));
    }
    if (lane == 0) R.U = __popcll(bal);
}

// Routing of the batch from the router logits inside one workgroup (all
// threads): top-k per token, slot table, first-appearance distinct slots.
__device__ void route_batch(const RouteArgs& a, RouteLds& R, int32_t* s_table, int32_t* s_first) {
    const int tid = threadIdx.x;
    const int T = a.T, k = a.k, npairs = a.npairs;
    if (tid == 0) R.bad = 0u;
    route_topk_dispatch(a.logits, T, a.E, k, a.norm, a.table, s_table, R);
    __syncthreads();
    VMI_STAMP(1, 1);
    if (npairs <= VMI_WAVE && a.cap <= kFirstTable) {
        if (tid < VMI_WAVE) slots_dedup_wave(a, R, s_table, s_first);
        __syncthreads();
        VMI_STAMP(1, 2);
        return;
    }
    if (tid < npairs) {
        const int id = R.ids[tid];
        int sl = (id >= 0 && id < a.E) ? (a.table ? s_table[id] : id) : -1;
        if (sl < 0 || sl >= a.cap) {
            sl = -1;
            atomicOr(&R.bad, VMI_STATUS_BAD_SLOT);
        }
        R.slot[tid] = sl;
    }
    __syncthreads();
    dedup_lds(npairs, k, a.cap, R, s_first);
    VMI_STAMP(1, 2);
}

// Routing of a caller's slot list (or pair p on matrix p without one).
__device__ void route_slots(const RouteArgs& a, RouteLds& R, int32_t* s_first) {
    const int tid = threadIdx.x;
    if (tid == 0) R.bad = 0u;
    __syncthreads();
    if (tid < a.npairs) {
        const int s = a.slots ? a.slots[tid] : tid;
        const bool ok = s >= 0 && s < a.cap;
        R.slot[tid] = ok ? s : -1;
        R.scores[tid] = a.in_scores[tid];
        if (!ok) atomicOr(&R.bad, VMI_STATUS_BAD_SLOT);
    }
    __syncthreads();
    dedup_lds(a.npairs, a.k, a.cap, R, s_first);
}

// The route table for the later kernels, the caller's ids/scores and the
// status bits, written by one routed workgroup once its own work is issued
// (nothing in the same kernel reads them).  pv[p] = 1 marks pair p as the
// first pair of its token on a valid slot: the pair whose rows carry that
// slot's contribution to the token.
__device__ void publish_route(const RouteArgs& a, const RouteLds& R) {
    const int tid = threadIdx.x;
    const int T = a.T, k = a.k, npairs = a.npairs;
    const int U = R.U;
    if (tid == 0) a.route->U = U;
    if (tid < npairs) {
        a.route->uslot[tid] = tid < U ? R.uslot[tid] : -1;
        const int s = R.slot[tid], t0 = (tid / k) * k;
        bool first = s >= 0;
        for (int p = t0; p < tid; ++p) first = first && R.slot[p] != s;
        a.route->pv[tid] = first ? 1 : 0;
    }
    // combine weight of (u, t): its pairs' scores in j order; rank of its first pair
    for (int i = tid; i < U * T; i += kThreads) {
        const int u = i / T, t = i - u * T;
        const int s = R.uslot[u];
        float wsum = 0.0f;
        int jr = -1;
        for (int j = 0; j < k; ++j)
            if (R.slot[t * k + j] == s) {
                wsum += R.scores[t * k + j];
                if (jr < 0) jr = j;
            }
        a.route->wt[u][t] = wsum;
        a.route->jr[u][t] = jr;
    }
    if (tid < npairs && !a.from_slots) {
        if (a.ids_out) a.ids_out[tid] = R.ids[tid];
        if (a.scores_out) a.scores_out[tid] = R.scores[tid];
    }
    if (tid == 0 && R.bad) atomicOr(a.status, R.bad);
}

struct ExpertArgs {
    RouteArgs ra;
    int has_shared, has_sgate;
    vmi_qmat gate, up, sh_gate, sh_up;
    vmi_qmat down, sh_down;       // group-major [n, I/64, H, 8 words], scales/biases [n, I/64, H]
    const vmi_u4* xop;            // [T, H/8]
    const float* xsum;            // [T, H/64]
    const float* fscale;          // [T]
    const float* sg_logit;        // [T] (has_sgate)
    uint16_t* part;               // [npairs + T, I/64, H] weighted partial rows, bf16
};

// One workgroup (4 waves) per item = blockIdx.x = u*NC + c: distinct slot u's
// slice c for u < U, the shared expert's slices at u = U (when present);
// workgroups past those exit after routing.  Every workgroup routes first:
// a CU then never holds one workgroup streaming weights while another waits
// for its router logits behind them (a CU returns loads in issue order, and
// workgroup 256 + j shares the CU of workgroup j).
//
// Gate/up: wave w owns rows c*64 + 16w + (lane % 16) of gate and up; lane
// block q = lane/16 loads 16 bytes at 64m + 16q of its row for m = 0..NM-1
// (two quantisation groups per m).  SwiGLU of the slice's 64 rows into LDS.
//
// Down (split over the intermediate dimension): the slice's 64 activations
// are exactly quantisation group c of the down projection's input, so the
// workgroup projects them through that group's column strip of every down
// row - H rows x 32 bytes, contiguous in the group-major pool - and writes
// one weighted fp32 partial row per (token, slice).  Wave w takes rows
// w*H/4 + 16b + r (b < H/64); lane (q, r) reads bytes 8q..8q+7 of row r of
// block b, so a wave's load covers 512 contiguous bytes.  The strip's loads
// are issued two blocks per gate/up step, into the registers the step frees.
// MFMA (v_mfma_f32_16x16x32_bf16, A = weights as exact bf16 128 + n, B =
// activations, D[4q + e][r] = row 4q + e of the block, token r): MFMA 0 takes
// dword 2q of each row (columns 16q..16q+7), MFMA 1 dword 2q + 1
// (16q+8..16q+15), and the activation operands follow that column order.
// Per row and token y = s (D - 128 X) + b X with X the token's activation
// sum over the group; the partial is y times the token's combine weight (the
// shared expert: its sigmoid gate).  Only token columns r < TB of D are
// real, so PF = 16 / TB blocks are packed into one register set by DPP row
// shifts first (block i's columns move to lanes r + i TB): the arithmetic and
// the stores then use every lane.
template <int NM, int TB>
__global__ __launch_bounds__(kThreads, TB <= 8 ? 2 : 1) void k_experts(ExpertArgs a) {
    constexpr bool PACK = TB <= 8;  // tokens of the even and odd groups share one gate/up MFMA
    constexpr int kT = PACK ? 8 : 16;
    constexpr int PF = 16 / TB;     // down blocks whose token columns share one register set
    constexpr int H = NM * 128, H8 = H / 8, NG = H / 64;
    constexpr int NB = NM / 4;      // bias MFMAs of 8 groups each
    constexpr int XPT = (kT * H8 + kThreads - 1) / kThreads;
    constexpr int RPW = H / 4;      // down rows per wave
    constexpr int NBW = RPW / 16;   // 16-row down blocks per wave (2 per gate/up step)
    constexpr int NDMA = H / 256;   // LDS copies of the strip's scales and biases (64 x 16 bytes each)
    static_assert(NBW == 2 * NM, "two down blocks per gate/up step");
    __shared__ vmi_u4 s_x[kT][H8 + 1];
    __shared__ float s_xs[kT][NG];
    __shared__ float s_inv[kT];
    __shared__ float s_act[kT][kSlice + 1];
    __shared__ __align__(16) uint32_t s_gus[2][kSlice][NG / 2];  // gate, up scales of the slice's rows (bf16 pairs)
    __shared__ __align__(16) uint16_t s_dsb[2][H];  // the strip's scales, then biases (bf16)
    __shared__ int32_t s_prow[kMaxT];
    __shared__ float s_wt[kMaxT];
    __shared__ RouteLds R;
    __shared__ int32_t s_table[kMaxE];
    __shared__ int32_t s_first[kFirstTable];
    const int tid = threadIdx.x, lane = tid & 63, w = vmi_wave_id();
    const int q = lane >> 4, r = lane & 15;
    const int T = a.ra.T, I = a.ra.I, k = a.ra.k, NC = I / kSlice;
    const int item = blockIdx.x;
    const vmi_u4 zero4 = {0u, 0u, 0u, 0u};
    VMI_STAMP(1, 0);
    VMI_STAMP_HWID(1, 5);
    // every argument in SGPRs at once (one scalar round trip)
    asm volatile("" ::"s"(a.ra.T), "s"(a.ra.I), "s"(a.ra.k), "s"(a.ra.E), "s"(a.ra.npairs), "s"(a.ra.norm),
                 "s"(a.ra.cap), "s"(a.ra.logits), "s"(a.ra.table), "s"(a.ra.route), "s"(a.ra.status));
    asm volatile("" ::"s"(a.ra.ids_out), "s"(a.ra.scores_out), "s"(a.has_shared), "s"(a.has_sgate), "s"(a.gate.w),
                 "s"(a.gate.s), "s"(a.gate.b), "s"(a.up.w), "s"(a.up.s), "s"(a.up.b));
    asm volatile("" ::"s"(a.sh_gate.w), "s"(a.sh_gate.s), "s"(a.sh_gate.b), "s"(a.sh_up.w), "s"(a.sh_up.s),
                 "s"(a.sh_up.b), "s"(a.down.w), "s"(a.down.s), "s"(a.down.b), "s"(a.sh_down.w));
    asm volatile("" ::"s"(a.sh_down.s), "s"(a.sh_down.b), "s"(a.xop), "s"(a.xsum), "s"(a.fscale), "s"(a.sg_logit),
                 "s"(a.part));

    // the MoE input operands do not depend on the routing: issued before it,
    // so their latency overlaps the router logits'
    const __amdgpu_buffer_rsrc_t rxo = vmi_rsrc(a.xop, (uint32_t)T * H8 * 16u);
    vmi_u4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) xr[i] = vmi_bload_b128(rxo, (uint32_t)(tid + kThreads * i) * 16u, 0);
    constexpr int XSPT = (kT * NG + kThreads - 1) / kThreads;
    const __amdgpu_buffer_rsrc_t rxs = vmi_rsrc(a.xsum, (uint32_t)T * NG * 4u);
    uint32_t xsr[XSPT];
#pragma unroll
    for (int i = 0; i < XSPT; ++i) xsr[i] = vmi_bload_b32(rxs, (uint32_t)(tid + kThreads * i) * 4u, 0);
    const uint32_t fsr = vmi_bload_b32(vmi_rsrc(a.fscale, (uint32_t)T * 4u), (uint32_t)tid * 4u, 0);
    const uint32_t sgr = vmi_bload_b32(vmi_rsrc(a.sg_logit, a.has_sgate ? (uint32_t)T * 4u : 0u), (uint32_t)tid * 4u, 0);

    route_batch(a.ra, R, s_table, s_first);
    const int u = item / NC, c = item - u * NC;
    const int U = vmi_uniform(R.U);
    const bool is_shared = u == U;
    if (u > U || (is_shared && !a.has_shared)) {
        if (item == 0) publish_route(a.ra, R);  // no item to compute at all
        return;
    }
    const int slot = is_shared ? 0 : vmi_uniform(R.uslot[u]);
    const uint32_t tmask = is_shared ? (1u << T) - 1u : (uint32_t)vmi_uniform((int)R.umask[u]);

    // every gate/up weight load of the item (scales, biases, words by m):
    // loads retire in issue order, so everything the arithmetic needs first is
    // issued first
    const vmi_qmat mg = is_shared ? a.sh_gate : a.gate;
    const vmi_qmat mu = is_shared ? a.sh_up : a.up;
    const uint32_t wbytes = (uint32_t)I * (H / 2), sbytes = (uint32_t)I * NG * 2u;
    const __amdgpu_buffer_rsrc_t rgw = vmi_rsrc(mg.w + (size_t)slot * I * H8, wbytes);
    const __amdgpu_buffer_rsrc_t ruw = vmi_rsrc(mu.w + (size_t)slot * I * H8, wbytes);
    const __amdgpu_buffer_rsrc_t rgb = vmi_rsrc(mg.b + (size_t)slot * I * NG, sbytes);
    const __amdgpu_buffer_rsrc_t rub = vmi_rsrc(mu.b + (size_t)slot * I * NG, sbytes);
    const uint32_t row = (uint32_t)(c * kSlice + 16 * w + r);
    const uint32_t sboff = row * NG * 2u;
    // the slice's gate and up scales straight into LDS (64 rows x NG bf16
    // each, contiguous): copy i (wave i % 4) moves 16-byte units 64i..64i+63
    {
        constexpr int NSC = 2 * kSlice * NG * 2 / 1024;  // 1 KB copies
        constexpr int UPM = kSlice * NG * 2 / 16;          // units per matrix
#pragma unroll
        for (int i = w; i < NSC; i += 4) {
            const int u = 64 * i + lane, x = u / UPM, o = u - x * UPM;
            vmi_lds_dma16_opaque_nt(reinterpret_cast<const uint8_t*>((x ? mu.s : mg.s) + ((size_t)slot * I + c * kSlice) * NG) + 16 * o,
                                    &s_gus[0][0][0] + 256 * i);
        }
    }
    uint32_t bgw[NB], buw[NB];
    {
        const uint32_t boff = sboff + 4u * NB * q;
        if constexpr (NB == 4) {
            const vmi_u4 g = vmi_bload_b128_nt(rgb, boff, 0), u = vmi_bload_b128_nt(rub, boff, 0);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                bgw[b] = g[b];
                buw[b] = u[b];
            }
        } else if constexpr (NB == 2) {
            const uint2 g = vmi_bload_b64_nt(rgb, boff, 0), u = vmi_bload_b64_nt(rub, boff, 0);
            bgw[0] = g.x; bgw[1] = g.y;
            buw[0] = u.x; buw[1] = u.y;
        } else {
            bgw[0] = vmi_bload_b32_nt(rgb, boff, 0);
            buw[0] = vmi_bload_b32_nt(rub, boff, 0);
        }
    }
    // Gate/up words in MFMA operand order (the pool is MFMA-major): block
    // (c, w, m) of a slot's matrix holds lane l's 16 bytes at 16 l, so each
    // wave load is 1 KB of contiguous memory and a slice 64 KB.
    vmi_u4 wl[2][NM];
    {
        const uint32_t woff = (uint32_t)((c * 4 + w) * NM) * 1024u + 16u * (uint32_t)lane;
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            wl[0][m] = vmi_bload_b128_nt(rgw, woff, 1024u * m);
            wl[1][m] = vmi_bload_b128_nt(ruw, woff, 1024u * m);
        }
    }
    // the down strip of this slice: rows of 32 bytes, group-major
    const vmi_qmat md = is_shared ? a.sh_down : a.down;
    const size_t drow0 = ((size_t)slot * NC + c) * H;
    const __amdgpu_buffer_rsrc_t rdw = vmi_rsrc(md.w + drow0 * 8, (uint32_t)H * 32u);
    const uint32_t doff = (uint32_t)(RPW * w + r) * 32u + 8u * (uint32_t)q;
    uint2 dw[NBW];

    // the first workgroup publishes the route while its weights stream
    if (item == 0) publish_route(a.ra, R);
    // partial row and combine weight of each token: a routed token's first
    // pair on this slot and the sum of its pairs' scores there; the shared
    // expert's rows follow the pairs, weighted by its sigmoid gate
    if (tid < T) {
        int pr = -1;
        float wt = 0.0f;
        if (is_shared) {
            pr = a.ra.npairs + tid;
            wt = a.has_sgate ? 1.0f / (1.0f + expf(-__uint_as_float(sgr))) : 1.0f;
        } else {
            for (int j = 0; j < k; ++j)
                if (R.slot[tid * k + j] == slot) {
                    wt += R.scores[tid * k + j];
                    if (pr < 0) pr = tid * k + j;
                }
        }
        s_prow[tid] = pr;
        s_wt[tid] = wt;
    }

    // operands into LDS
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const int idx = tid + kThreads * i;
        if (idx < T * H8) s_x[idx / H8][idx % H8] = xr[i];
    }
#pragma unroll
    for (int i = 0; i < XSPT; ++i) {
        const int idx = tid + kThreads * i;
        if (idx < T * NG) s_xs[idx / NG][idx % NG] = __uint_as_float(xsr[i]);
    }
    if (tid < T) s_inv[tid] = 1.0f / __uint_as_float(fsr);
    // the scale copies precede the two bias loads and the 2 NM weight loads
    // (and, in one workgroup, the route's stores): with at most 2 + 2 NM
    // operations outstanding they have landed
    vmi_vm_wait_c<2 + 2 * NM>();
    __syncthreads();

    // affine-bias term first: its inputs (the x group sums and the bias words,
    // loaded ahead of every weight word) are already here, so it runs while
    // the weights stream rather than after them.  Lane block q carries groups
    // 2*NB*q + 2b, +1.
    const vmi_f4 zf = {0.0f, 0.0f, 0.0f, 0.0f};
    vmi_f4 bgd = zf, bud = zf;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int g0 = 2 * NB * q + 2 * b;
        const vmi_u4 ab = (r < T) ? vmi_bias_a_operand(s_xs[r][g0], s_xs[r][g0 + 1]) : zero4;
        bgd = vmi_mfma_bf16(ab, vmi_bias_b_operand(bgw[b]), bgd);
        bud = vmi_mfma_bf16(ab, vmi_bias_b_operand(buw[b]), bud);
    }

    // main MFMAs: m-th load pair covers groups 2m (K blocks 0-1) and 2m+1 (2-3)
    const int par = lane >> 5;  // PACK: D rows 8..15 (lanes 32..63) hold the odd group
    float accg[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accu[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // without PACK the odd groups accumulate apart and meet the even ones at the
    // end, as the two lane halves do with PACK: the same rounding for every T
    float accg1[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accu1[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const int tk = PACK ? (r & 7) : r;
    const bool xreal = PACK ? (((q < 2) == (r < 8)) && tk < T) : (r < T);
    const int tkc = tk < T ? tk : 0;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        const vmi_u4 wgm = wl[0][m], wum = wl[1][m];
        vmi_u4 ax[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const vmi_u4 v = s_x[tkc][16 * m + 4 * q + j];
            ax[j] = xreal ? v : zero4;
        }
        const uint32_t swg = s_gus[0][16 * w + r][m], swu = s_gus[1][16 * w + r][m];
        if constexpr (PACK) {
            vmi_f4 dg = zf, du = zf;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dg = vmi_mfma_f16(ax[j], vmi_unpack_u4_f16(wgm[j]), dg);
                du = vmi_mfma_f16(ax[j], vmi_unpack_u4_f16(wum[j]), du);
            }
            const float sgf = __uint_as_float(par ? (swg & 0xffff0000u) : (swg << 16));
            const float suf = __uint_as_float(par ? (swu & 0xffff0000u) : (swu << 16));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                accg[e] = fmaf(sgf, dg[e], accg[e]);
                accu[e] = fmaf(suf, du[e], accu[e]);
            }
        } else {
            vmi_f4 dg0 = zf, du0 = zf, dg1 = zf, du1 = zf;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const vmi_u4 a0 = q < 2 ? ax[j] : zero4, a1 = q < 2 ? zero4 : ax[j];
                const vmi_u4 bg = vmi_unpack_u4_f16(wgm[j]), bu = vmi_unpack_u4_f16(wum[j]);
                dg0 = vmi_mfma_f16(a0, bg, dg0);
                dg1 = vmi_mfma_f16(a1, bg, dg1);
                du0 = vmi_mfma_f16(a0, bu, du0);
                du1 = vmi_mfma_f16(a1, bu, du1);
            }
            const float sg0 = __uint_as_float(swg << 16), sg1 = __uint_as_float(swg & 0xffff0000u);
            const float su0 = __uint_as_float(swu << 16), su1 = __uint_as_float(swu & 0xffff0000u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                accg[e] = fmaf(sg0, dg0[e], accg[e]);
                accu[e] = fmaf(su0, du0[e], accu[e]);
                accg1[e] = fmaf(sg1, dg1[e], accg1[e]);
                accu1[e] = fmaf(su1, du1[e], accu1[e]);
            }
        }
        // the step's accumulators are settled here, so its MFMA results die
        // here (the scale FMAs are not sunk past the loop, which would hold
        // those results across it)
        asm volatile("" : "+v"(accg[0]), "+v"(accg[1]), "+v"(accg[2]), "+v"(accg[3]));
        asm volatile("" : "+v"(accu[0]), "+v"(accu[1]), "+v"(accu[2]), "+v"(accu[3]));
        if constexpr (!PACK) {
            asm volatile("" : "+v"(accg1[0]), "+v"(accg1[1]), "+v"(accg1[2]), "+v"(accg1[3]));
            asm volatile("" : "+v"(accu1[0]), "+v"(accu1[1]), "+v"(accu1[2]), "+v"(accu1[3]));
        }
        // two blocks of the down strip into the registers this step freed
        dw[2 * m] = vmi_bload_b64_nt(rdw, doff + 1024u * (uint32_t)m, 0);
        dw[2 * m + 1] = vmi_bload_b64_nt(rdw, doff + 1024u * (uint32_t)m + 512u, 0);
        // the strip's scales and biases straight into LDS (no registers held):
        // copy i (wave i % 4) moves 16-byte units 64i..64i+63 of [scales, biases]
        if (m == 0) {
#pragma unroll
            for (int i = w; i < NDMA; i += 4) {
                const int u = 64 * i + lane, arr = u / H8, o = u - arr * H8;
                vmi_lds_dma16_opaque_nt((arr ? md.b : md.s) + drow0 + 8 * o, &s_dsb[0][0] + 8 * 64 * i);
            }
        }
    }
    // the copies were issued after the first two strip loads: with at most
    // NBW - 2 operations outstanding they have landed (the barrier below then
    // publishes them to every wave)
    vmi_vm_wait_c<NBW - 2>();
    VMI_STAMP(1, 3);
    // SwiGLU of token t = 4*(lane/16) + e, row 16w + r of the slice
    const int tq = lane >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float tg = accg[e], tu = accu[e];
        if constexpr (PACK) {
            tg += __shfl_xor(tg, 32, VMI_WAVE);
            tu += __shfl_xor(tu, 32, VMI_WAVE);
        } else {
            tg += accg1[e];
            tu += accu1[e];
        }
        const int t = 4 * tq + e;
        if ((!PACK || tq < 2) && t < T) {
            const float inv = s_inv[t];
            const float g = fmaf(tg, kTwo24, bgd[e]) * inv;
            const float u = fmaf(tu, kTwo24, bud[e]) * inv;
            s_act[t][16 * w + r] = ((tmask >> t) & 1u) ? g * (1.0f / (1.0f + expf(-g))) * u : 0.0f;
        }
    }
    __syncthreads();
    VMI_STAMP(1, 4);

    // down: token r's 64 activations as bf16 B operands, and their sum X in
    // column order (each lane its 16 columns, then across the lane blocks)
    const bool tcol = r < T;
    vmi_u4 b0, b1;
    float X = 0.0f;
    {
        float av[16];
        const float* ar = &s_act[tcol ? r : 0][16 * q];
#pragma unroll
        for (int i = 0; i < 16; ++i) av[i] = tcol ? ar[i] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            b0[i] = vmi_pack_bf16x2(av[i], av[i + 4]);
            b1[i] = vmi_pack_bf16x2(av[8 + i], av[12 + i]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) X += __uint_as_float(b0[i] << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) X += __uint_as_float(b0[i] & 0xffff0000u);
#pragma unroll
        for (int i = 0; i < 4; ++i) X += __uint_as_float(b1[i] << 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) X += __uint_as_float(b1[i] & 0xffff0000u);
    }
    X += __shfl_xor(X, 16, VMI_WAVE);
    X += __shfl_xor(X, 32, VMI_WAVE);
    // the wave's rows' scale s and c = b - 128 s in fp32, into the x operand
    // buffer (every wave is past the gate/up MFMAs): y = s D + c X, as
    // s (D - 128 X) + b X for D = sum (128 + n) a
    float* scw = reinterpret_cast<float*>(&s_x[0][0]);  // s [H], then c [H]
    static_assert(sizeof(s_x) >= 2 * H * sizeof(float), "scales fit the operand buffer");
#pragma unroll
    for (int i = lane; i < RPW / 8; i += VMI_WAVE) {
        const int h8 = RPW * w + 8 * i;
        const vmi_u4 sv = *reinterpret_cast<const vmi_u4*>(&s_dsb[0][h8]);
        const vmi_u4 bv = *reinterpret_cast<const vmi_u4*>(&s_dsb[1][h8]);
        float sf[8], cf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sf[2 * j] = __uint_as_float(sv[j] << 16);
            sf[2 * j + 1] = __uint_as_float(sv[j] & 0xffff0000u);
            cf[2 * j] = fmaf(-128.0f, sf[2 * j], __uint_as_float(bv[j] << 16));
            cf[2 * j + 1] = fmaf(-128.0f, sf[2 * j + 1], __uint_as_float(bv[j] & 0xffff0000u));
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            *reinterpret_cast<float4*>(&scw[h8 + 4 * j]) = make_float4(sf[4 * j], sf[4 * j + 1], sf[4 * j + 2], sf[4 * j + 3]);
            *reinterpret_cast<float4*>(&scw[H + h8 + 4 * j]) = make_float4(cf[4 * j], cf[4 * j + 1], cf[4 * j + 2], cf[4 * j + 3]);
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // after packing, lane (q, r) holds token rt = r % TB of block r / TB: its
    // activation sum comes from lane (q, rt)
    const int rt = r % TB, pi = r / TB;
    const float Xp = __shfl(X, (lane & ~15) | rt, VMI_WAVE);
    const bool store = rt < T && ((tmask >> rt) & 1u);
    const float wt = store ? s_wt[rt] : 0.0f;
    const int prow = store ? s_prow[rt] : 0;
    // partial rows through a buffer resource: lanes without a row of theirs
    // store past its range, so the loop has no branch and the blocks' MFMAs
    // and arithmetic interleave
    const __amdgpu_buffer_rsrc_t rpart =
        vmi_rsrc(a.part, (uint32_t)((size_t)(a.ra.npairs + T) * NC * H * sizeof(uint16_t)));
    const uint32_t pbase =
        store ? (uint32_t)((((size_t)prow * NC + c) * H + RPW * w + 16 * pi + 4 * q) * sizeof(uint16_t)) : VMI_OOB;
    // (the strip's loads were all issued before the first store, so the counted
    // wait for a block never waits for a store)
    VMI_STAMP(1, 7);
    static_assert(NBW % PF == 0, "whole block packs");
#pragma unroll
    for (int bb = 0; bb < NBW; bb += PF) {
        if (bb == NBW / 2) VMI_STAMP(1, 8);
        vmi_f4 D[PF];
#pragma unroll
        for (int i = 0; i < PF; ++i) D[i] = vmi_mfma_bf16(vmi_unpack_u4_bf16_128(dw[bb + i].x), b0, zf);
#pragma unroll
        for (int i = 0; i < PF; ++i) D[i] = vmi_mfma_bf16(vmi_unpack_u4_bf16_128(dw[bb + i].y), b1, D[i]);
        vmi_f4 E = D[0];
        if constexpr (PF == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                E[e] = vmi_dpp_into<0x114, 0x2>(E[e], D[1][e]);  // row_shr:4 into lanes 4..7
                E[e] = vmi_dpp_into<0x118, 0x4>(E[e], D[2][e]);  // row_shr:8 into lanes 8..11
                E[e] = vmi_dpp_into<0x11C, 0x8>(E[e], D[3][e]);  // row_shr:12 into lanes 12..15
            }
        } else if constexpr (PF == 2) {
#pragma unroll
            for (int e = 0; e < 4; ++e) E[e] = vmi_dpp_into<0x118, 0xC>(E[e], D[1][e]);  // row_shr:8 into lanes 8..15
        }
        const int h = RPW * w + 16 * (bb + pi) + 4 * q;
        const float4 sv = *reinterpret_cast<const float4*>(&scw[h]);
        const float4 cv = *reinterpret_cast<const float4*>(&scw[H + h]);
        // the partial row rounded to bf16 (the reference's expert outputs are bf16)
        const uint2 o = make_uint2(vmi_pack_bf16x2(wt * fmaf(sv.x, E[0], cv.x * Xp), wt * fmaf(sv.y, E[1], cv.y * Xp)),
                                   vmi_pack_bf16x2(wt * fmaf(sv.z, E[2], cv.z * Xp), wt * fmaf(sv.w, E[3], cv.w * Xp)));
        vmi_bstore_b64(o, rpart, pbase, 32u * (uint32_t)bb);
    }
    VMI_STAMP(1, 6);
}

// ------------------------------------------------------------- combine
struct CombineArgs {
    int T, H, NC, k, npairs, has_shared;
    const RouteInfo* route;
    const uint16_t* part;      // [npairs + T, NC, H] bf16
    const uint16_t* residual;  // [T, H] or nullptr
    uint16_t* out;             // [T, H] bf16
};

constexpr int kCbRows = 8;  // output rows per combine workgroup

// One workgroup per 8 output rows h0..h0+7, the tiles of one XCD adjacent
// (workgroup i sits on XCD i % 8 and takes tile (i % 8) * (tiles / 8) + i / 8),
// so the 32-byte pieces of a partial row that neighbouring tiles read share
// that XCD's L2 lines.  Per token, in a fixed order: every pair's slices
// 0..NC-1, then the pairs in rank order (a pair without rows of its own - a
// repeated or invalid slot - adds nothing), the shared expert last, then the
// residual.  Nothing depends on the other tokens of the batch.
__global__ __launch_bounds__(kThreads) void k_moe_combine(CombineArgs a) {
    __shared__ float s_y[kMaxT][kMaxK + 1][kCbRows];
    const int tid = threadIdx.x;
    const int T = a.T, k = a.k, H = a.H, NC = a.NC;
    const int per = H / kCbRows / 8;
    const int tile = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    const int h0 = tile * kCbRows;
    VMI_STAMP(2, 0);
    asm volatile("" ::"s"(a.T), "s"(a.H), "s"(a.NC), "s"(a.k), "s"(a.npairs), "s"(a.has_shared), "s"(a.route),
                 "s"(a.part), "s"(a.residual), "s"(a.out));
    const bool fin = tid < T * kCbRows;
    const uint32_t resid_bits =
        vmi_bload_b16(vmi_rsrc(a.residual, a.residual ? (uint32_t)T * H * 2u : 0u),
                      fin ? (uint32_t)((tid >> 3) * H + h0 + (tid & 7)) * 2u : VMI_OOB, 0);
    // every item's flag and slices through buffer resources (slices past NC
    // and items past the batch read nothing), all requested before any wait;
    // T * (k + 1) * 2 <= 2 (160 + 16) items fit two passes of the workgroup
    const int nitem = T * (k + 1) * 2;
    const __amdgpu_buffer_rsrc_t rp = vmi_rsrc(a.part, (uint32_t)((size_t)(a.npairs + T) * NC * H * sizeof(uint16_t)));
    const __amdgpu_buffer_rsrc_t rf = vmi_rsrc(a.route->pv, (uint32_t)a.npairs * 4u);
    constexpr int MC = kMaxInter / kSlice;
    uint2 v[2][MC];
    uint32_t flag[2];
    int tj[2];
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int i = tid + kThreads * it;
        const bool ok = i < nitem;
        const int half = i & 1;
        tj[it] = ok ? i >> 1 : 0;
        const int t = tj[it] / (k + 1), j = tj[it] - t * (k + 1);
        const int p = j < k ? t * k + j : a.npairs + t;
        const uint32_t fl = vmi_bload_b32(rf, (ok && j < k) ? 4u * (uint32_t)p : VMI_OOB, 0);
        flag[it] = j < k ? fl : (uint32_t)(ok && a.has_shared);
        const uint32_t off = (uint32_t)(((size_t)p * NC * H + h0 + 4 * half) * sizeof(uint16_t));
#pragma unroll
        for (int cc = 0; cc < MC; ++cc)
            v[it][cc] = vmi_bload_b64(rp, (ok && cc < NC) ? off + (uint32_t)(cc * H * sizeof(uint16_t)) : VMI_OOB, 0);
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int i = tid + kThreads * it;
        if (i < nitem) {
            const int half = i & 1, t = tj[it] / (k + 1), j = tj[it] - t * (k + 1);
            float y[4] = {__uint_as_float(v[it][0].x << 16), __uint_as_float(v[it][0].x & 0xffff0000u),
                          __uint_as_float(v[it][0].y << 16), __uint_as_float(v[it][0].y & 0xffff0000u)};
#pragma unroll
            for (int cc = 1; cc < MC; ++cc)
                if (cc < NC) {
                    y[0] += __uint_as_float(v[it][cc].x << 16);
                    y[1] += __uint_as_float(v[it][cc].x & 0xffff0000u);
                    y[2] += __uint_as_float(v[it][cc].y << 16);
                    y[3] += __uint_as_float(v[it][cc].y & 0xffff0000u);
                }
            *reinterpret_cast<float4*>(&s_y[t][j][4 * half]) =
                flag[it] ? make_float4(y[0], y[1], y[2], y[3]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    __syncthreads();
    if (fin) {
        const int t = tid >> 3, rr = tid & 7;
        float acc = 0.0f;
        for (int j = 0; j <= k; ++j) acc += s_y[t][j][rr];
        acc += vmi_bf16_to_f32(resid_bits);
        a.out[(size_t)t * H + h0 + rr] = vmi_f32_to_bf16(acc);
    }
    VMI_STAMP(2, 1);
}

// ------------------------------------------------- fp32 operator path
// vmi_fused_moe_slots / vmi_fused_moe_staged keep the reference operator's
// fp32 arithmetic (fused_moe.cpp:221-298: fp32 x - bf16 x is widened exactly
// when staged, as the reference's caller casts it, native_moe.py:481 - fp32
// dequantised weights, fp32 activations, reduce_pairs over j in order).  Each 16-byte
// chunk of a weight row holds 32 columns of one quantisation group, so the
// affine dequantisation q*s + b is factored out of the chunk's sum:
//   sum_c (q_c s + b) x_c = s * sum_c q_c x_c + b * sum_c x_c,
// with both sums in fp32 (the 4-bit values are exact, the products rounded
// once each), then the chunks of a row are added across the lanes that hold
// them.  Three launches: gate/up + SwiGLU per (distinct slot, 32 rows of I)
// into fp32 activation rows, down per (distinct slot, rows of H) into one
// fp32 output row per (token, distinct slot), and the combine per (t, h).

constexpr int kFTok = 4;  // token rows per LDS chunk
// Staged rows keep each 32-column chunk 36 floats apart, so the eight lanes
// reading eight consecutive chunks of one row start on different LDS banks.
constexpr int kFChunk = 36;

// Lane geometry of a weight row of LEN columns (LEN a multiple of 64): LPR
// lanes share a row, each taking NI 16-byte chunks; a wave covers RPW rows
// and a 256-thread workgroup RPB.
template <int LEN>
struct FRow {
    static constexpr int NHG = LEN / 32;  // 32-column chunks (half groups)
    static constexpr int LPR = NHG % 8 == 0 ? 8 : (NHG % 4 == 0 ? 4 : 2);
    static constexpr int NI = NHG / LPR;
    static constexpr int RPW = VMI_WAVE / LPR;
    static constexpr int RPB = (kThreads / VMI_WAVE) * RPW;
};

// sum_c q_c x_c over the 32 columns of one 16-byte chunk; xs points at the
// chunk's first column in LDS.
__device__ __forceinline__ float dot32_u4_f32(const vmi_u4& wv, const float* xs) {
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        uint32_t word = wv[m];
        asm volatile("" : "+v"(word));
        const float4 x0 = *reinterpret_cast<const float4*>(xs + 8 * m);
        const float4 x1 = *reinterpret_cast<const float4*>(xs + 8 * m + 4);
        acc = fmaf((float)(word & 15u), x0.x, acc);
        acc = fmaf((float)((word >> 4) & 15u), x0.y, acc);
        acc = fmaf((float)((word >> 8) & 15u), x0.z, acc);
        acc = fmaf((float)((word >> 12) & 15u), x0.w, acc);
        acc = fmaf((float)((word >> 16) & 15u), x1.x, acc);
        acc = fmaf((float)((word >> 20) & 15u), x1.y, acc);
        acc = fmaf((float)((word >> 24) & 15u), x1.z, acc);
        acc = fmaf((float)(word >> 28), x1.w, acc);
    }
    return acc;
}

// Rows src + ridx[j] * LEN (j < kFTok, ridx < 0: zeros) into s[j] (chunk hg
// at kFChunk * hg), then the fp32 sum of every 32-column chunk into sh[j].
// All threads; ends synced.
__device__ __forceinline__ float4 load_f4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float4 load_f4(const uint16_t* p) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                       __uint_as_float(v.y & 0xffff0000u));
}

template <int LEN, typename XT>
__device__ __forceinline__ void stage_rows_f32(const XT* __restrict__ src, const int (&ridx)[kFTok],
                                               float (*s)[LEN / 32 * kFChunk], float (*sh)[LEN / 32]) {
    const int tid = threadIdx.x;
    __syncthreads();  // the previous chunk's readers are done
    for (int i = tid; i < kFTok * (LEN / 4); i += kThreads) {
        const int j = i / (LEN / 4), c4 = i - j * (LEN / 4);
        float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (ridx[j] >= 0) v = load_f4(src + (size_t)ridx[j] * LEN + 4 * c4);
        *reinterpret_cast<float4*>(&s[j][kFChunk * (c4 >> 3) + 4 * (c4 & 7)]) = v;
    }
    __syncthreads();
    for (int i = tid; i < kFTok * (LEN / 32); i += kThreads) {
        const int j = i / (LEN / 32), hg = i - j * (LEN / 32);
        const float* xs = &s[j][kFChunk * hg];
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < 32; c += 4) {
            const float4 v = *reinterpret_cast<const float4*>(xs + c);
            acc += v.x;
            acc += v.y;
            acc += v.z;
            acc += v.w;
        }
        sh[j][hg] = acc;
    }
    __syncthreads();
}

// One lane's share of a row times staged row j: its NI chunks, each
// s * (q . x) + b * (x sum), then the row total over the LPR lanes.
template <int LEN>
__device__ __forceinline__ float row_dot_f32(const vmi_u4 (&wv)[FRow<LEN>::NI], const float (&sc)[FRow<LEN>::NI],
                                             const float (&bi)[FRow<LEN>::NI], const float* s_row,
                                             const float* sh_row, int part) {
    using G = FRow<LEN>;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
        const int hg = G::LPR * i + part;
        const float d = dot32_u4_f32(wv[i], s_row + kFChunk * hg);
        acc = fmaf(sc[i], d, acc);
        acc = fmaf(bi[i], sh_row[hg], acc);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int o = 1; o < G::LPR; o <<= 1) acc += __shfl_xor(acc, o, VMI_WAVE);
    return acc;
}

// row_dot_f32 of two matrices' rows (gate and up) over the same staged row,
// chunk by chunk, so that each chunk of x is read from LDS once.
template <int LEN>
__device__ __forceinline__ void row_dot2_f32(const vmi_u4 (&w0)[FRow<LEN>::NI], const float (&s0)[FRow<LEN>::NI],
                                             const float (&b0)[FRow<LEN>::NI], const vmi_u4 (&w1)[FRow<LEN>::NI],
                                             const float (&s1)[FRow<LEN>::NI], const float (&b1)[FRow<LEN>::NI],
                                             const float* s_row, const float* sh_row, int part, float& r0,
                                             float& r1) {
    using G = FRow<LEN>;
    float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
        const int hg = G::LPR * i + part;
        const float* xs = s_row + kFChunk * hg;
        float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t u0 = w0[i][m], u1 = w1[i][m];
            // opaque per call: keeps the compiler from converting every
            // weight once, ahead of the token loop, into 64 * NI registers
            asm volatile("" : "+v"(u0), "+v"(u1));
            const float4 x0 = *reinterpret_cast<const float4*>(xs + 8 * m);
            const float4 x1 = *reinterpret_cast<const float4*>(xs + 8 * m + 4);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int n = 0; n < 8; ++n) {
                d0 = fmaf((float)((u0 >> (4 * n)) & 15u), xv[n], d0);
                d1 = fmaf((float)((u1 >> (4 * n)) & 15u), xv[n], d1);
            }
        }
        const float xh = sh_row[hg];
        a0 = fmaf(s0[i], d0, a0);
        a0 = fmaf(b0[i], xh, a0);
        a1 = fmaf(s1[i], d1, a1);
        a1 = fmaf(b1[i], xh, a1);
        // one chunk of x in registers at a time (hoisting every chunk's LDS
        // reads ahead of the arithmetic would need 8 * NI registers a lane)
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int o = 1; o < G::LPR; o <<= 1) {
        a0 += __shfl_xor(a0, o, VMI_WAVE);
        a1 += __shfl_xor(a1, o, VMI_WAVE);
    }
    r0 = a0;
    r1 = a1;
}

// Weights, scales and biases of row `row` of matrix `mat` (uniform) of a
// stack of rows x LEN matrices, the lane's NI chunks (chunk i at column
// 32 * (LPR * i + part)).  The buffer resources span the whole matrix, so
// they stay uniform; the row is in the per-lane offset.
template <int LEN>
__device__ __forceinline__ void load_row_f32(const vmi_qmat& m, int mat, int rows, int row, int part,
                                             vmi_u4 (&wv)[FRow<LEN>::NI], float (&sc)[FRow<LEN>::NI],
                                             float (&bi)[FRow<LEN>::NI]) {
    using G = FRow<LEN>;
    constexpr int NG = LEN / 64;
    const size_t m0 = (size_t)mat * rows;
    const __amdgpu_buffer_rsrc_t rw = vmi_rsrc(m.w + m0 * (LEN / 8), (uint32_t)rows * (LEN / 2));
    const __amdgpu_buffer_rsrc_t rs = vmi_rsrc(m.s + m0 * NG, (uint32_t)rows * NG * 2);
    const __amdgpu_buffer_rsrc_t rb = vmi_rsrc(m.b + m0 * NG, (uint32_t)rows * NG * 2);
    const uint32_t wrow = (uint32_t)row * (LEN / 2), srow = (uint32_t)row * NG * 2;
#pragma unroll
    for (int i = 0; i < G::NI; ++i) {
        const int hg = G::LPR * i + part;
        wv[i] = vmi_bload_b128_nt(rw, wrow + 16u * hg, 0);
        sc[i] = __uint_as_float(vmi_bload_b16(rs, srow + 2u * (hg >> 1), 0) << 16);
        bi[i] = __uint_as_float(vmi_bload_b16(rb, srow + 2u * (hg >> 1), 0) << 16);
    }
}

// Gate/up + SwiGLU.  Item blockIdx.x = u * (I / RPB) + c: rows c*RPB.. of
// distinct slot u's gate and up matrices for the tokens routed to it, in
// chunks of kFTok tokens.  act row t*k + j (j the token's first rank on the
// slot) receives the token's activations.  The first workgroup publishes the
// route and prow[p] = the activation/output row of pair p (-1: bad slot).
struct F32Args {
    RouteArgs ra;
    vmi_qmat gate, up;
};

template <int H, typename XT>
__global__ __launch_bounds__(kThreads) void k_gateup_f32(F32Args fa, const XT* __restrict__ x,
                                                         float* __restrict__ act, int32_t* __restrict__ prow) {
    const RouteArgs& a = fa.ra;
    using G = FRow<H>;
    __shared__ float s_x[kFTok][H / 32 * kFChunk];
    __shared__ float s_h[kFTok][H / 32];
    __shared__ RouteLds R;
    __shared__ int32_t s_first[kFirstTable];
    const int tid = threadIdx.x, lane = tid & 63, w = vmi_wave_id();
    const int part = lane % G::LPR, rr = lane / G::LPR;
    const int I = a.I, NC = I / G::RPB, k = a.k;
    route_slots(a, R, s_first);
    const int item = blockIdx.x, u = item / NC, c = item - u * NC;
    if (item == 0) {
        publish_route(a, R);
        if (tid < a.npairs) {
            const int sl = R.slot[tid], t = tid / k;
            int pr = -1;
            if (sl >= 0)
                for (int j = 0; j < k; ++j)
                    if (R.slot[t * k + j] == sl) {
                        pr = t * k + j;
                        break;
                    }
            prow[tid] = pr;
        }
    }
    if (u >= vmi_uniform(R.U)) return;
    const int slot = vmi_uniform(R.uslot[u]);
    uint32_t tmask = (uint32_t)vmi_uniform((int)R.umask[u]);
    const int row = c * G::RPB + G::RPW * w + rr;

    vmi_u4 gw[G::NI], uw[G::NI];
    float gs[G::NI], gb[G::NI], us[G::NI], ub[G::NI];
    load_row_f32<H>(fa.gate, slot, I, row, part, gw, gs, gb);
    load_row_f32<H>(fa.up, slot, I, row, part, uw, us, ub);

    while (tmask) {  // uniform: chunks of up to kFTok of the slot's tokens
        int ridx[kFTok];
#pragma unroll
        for (int j = 0; j < kFTok; ++j) {
            ridx[j] = tmask ? __builtin_ctz(tmask) : -1;
            tmask &= tmask ? tmask - 1u : 0u;
        }
        stage_rows_f32<H, XT>(x, ridx, s_x, s_h);
#pragma unroll 1
        for (int j = 0; j < kFTok; ++j) {
            if (ridx[j] < 0) break;
            float g, v;
            row_dot2_f32<H>(gw, gs, gb, uw, us, ub, s_x[j], s_h[j], part, g, v);
            if (part == 0) {
                const int t = ridx[j];
                int pr = t * k;
                for (int jj = 0; jj < k; ++jj)
                    if (R.slot[t * k + jj] == slot) {
                        pr = t * k + jj;
                        break;
                    }
                act[(size_t)pr * I + row] = g * (1.0f / (1.0f + expf(-g))) * v;
            }
        }
    }
}

// Down projection.  Item blockIdx.x = u * (H / RPB) + c: rows c*RPB.. of
// distinct slot u's down matrix times the activation row of every token
// routed to it, into output row t*k + jr[u][t].
template <int I>
__global__ __launch_bounds__(kThreads) void k_down_f32(const RouteInfo* __restrict__ route, vmi_qmat down, int T,
                                                       int k, int H, const float* __restrict__ act,
                                                       float* __restrict__ y) {
    using G = FRow<I>;
    __shared__ float s_a[kFTok][I / 32 * kFChunk];
    __shared__ float s_h[kFTok][I / 32];
    const int tid = threadIdx.x, lane = tid & 63, w = vmi_wave_id();
    const int part = lane % G::LPR, rr = lane / G::LPR;
    const int NC = H / G::RPB;
    const int item = blockIdx.x, u = item / NC, c = item - u * NC;
    if (u >= vmi_uniform(route->U)) return;
    const int slot = vmi_uniform(route->uslot[u]);
    const int row = c * G::RPB + G::RPW * w + rr;
    vmi_u4 dw[G::NI];
    float ds[G::NI], db[G::NI];
    load_row_f32<I>(down, slot, H, row, part, dw, ds, db);
    int t0 = 0;
    while (true) {  // uniform: the next kFTok tokens with a pair on u
        int ridx[kFTok], orow[kFTok];
        int n = 0;
        for (; t0 < T && n < kFTok; ++t0) {
            const int jr = route->jr[u][t0];
            if (jr >= 0) {
                ridx[n] = t0 * k + jr;
                orow[n] = ridx[n];
                ++n;
            }
        }
        if (n == 0) break;
        for (int j = n; j < kFTok; ++j) ridx[j] = orow[j] = -1;
        stage_rows_f32<I, float>(act, ridx, s_a, s_h);
#pragma unroll 1
        for (int j = 0; j < kFTok; ++j) {
            if (orow[j] < 0) break;
            const float v = row_dot_f32<I>(dw, ds, db, s_a[j], s_h[j], part);
            if (part == 0) y[(size_t)orow[j] * H + row] = v;
        }
    }
}

// out[t][h] = sum over j in order of y[prow[t*k+j]][h] * scores[t*k+j]
// (reduce_pairs, fused_moe.cpp:286-298); a pair with a bad slot adds nothing.
__global__ __launch_bounds__(kThreads) void k_combine_f32(const int32_t* __restrict__ prow,
                                                          const float* __restrict__ scores,
                                                          const float* __restrict__ y, int T, int k, int H,
                                                          void* out, int out_dtype) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= T * H) return;
    const int t = i / H, h = i - t * H;
    float acc = 0.0f;
    for (int j = 0; j < k; ++j) {
        const int pr = prow[t * k + j];
        if (pr >= 0) acc += y[(size_t)pr * H + h] * scores[t * k + j];
    }
    if (out_dtype == VMI_F32)
        reinterpret_cast<float*>(out)[i] = acc;
    else
        reinterpret_cast<uint16_t*>(out)[i] = vmi_f32_to_bf16(acc);
}

// ---------------------------------------------------------------- host
bool aligned(const void* p, size_t n) { return ((uintptr_t)p % n) == 0; }

bool qmat_ok(const vmi_qmat& m) { return m.w && m.s && m.b && aligned(m.w, 16) && aligned(m.s, 16) && aligned(m.b, 16); }

int check_shape(int T, int k, int hidden, int inter, int group, int bits) {
    if (T <= 0 || k <= 0) return vmi::fail(VMI_ERR_INVALID, "T=%d and k=%d must be positive", T, k);
    if (T > kMaxT) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d exceeds %d (verify batch limit)", T, kMaxT);
    if (T * k > kMaxPairs) return vmi::fail(VMI_ERR_UNSUPPORTED, "T*k=%d exceeds %d", T * k, kMaxPairs);
    if (k > kMaxK) return vmi::fail(VMI_ERR_UNSUPPORTED, "k=%d exceeds %d", k, kMaxK);
    if (bits != 4 || group != 64)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "only bits=4, group=64 is built (got bits=%d group=%d)", bits, group);
    if (hidden != 512 && hidden != 1024 && hidden != 2048)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d not in {512,1024,2048}", hidden);
    if (inter % kSlice || inter < kSlice || inter > kMaxInter)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "inter=%d must be a multiple of 64 up to %d", inter, kMaxInter);
    return VMI_OK;
}

template <int TB>
hipError_t launch_experts_t(const ExpertArgs& ea, int H, hipStream_t s) {
    const int NC = ea.ra.I / kSlice;
    const dim3 grid((ea.has_shared ? NC : 0) + ea.ra.npairs * NC);
    switch (H) {
        case 512: hipLaunchKernelGGL((k_experts<4, TB>), grid, dim3(kThreads), 0, s, ea); break;
        case 1024: hipLaunchKernelGGL((k_experts<8, TB>), grid, dim3(kThreads), 0, s, ea); break;
        default: hipLaunchKernelGGL((k_experts<16, TB>), grid, dim3(kThreads), 0, s, ea); break;
    }
    return hipGetLastError();
}

// token blocks of 4, 8 or 16: the batch's tokens fill that many MFMA columns
hipError_t launch_experts(const ExpertArgs& ea, int H, hipStream_t s) {
    if (ea.ra.T <= 4) return launch_experts_t<4>(ea, H, s);
    if (ea.ra.T <= 8) return launch_experts_t<8>(ea, H, s);
    return launch_experts_t<16>(ea, H, s);
}

// Workspace of the fp32 operator path: the status word and route table at the
// offsets carve_workspace gives them, then the pair rows.
struct F32Workspace {
    uint32_t* status;
    RouteInfo* route;
    int32_t* prow;  // [T*k]
    float* act;     // [T*k, I]
    float* y;       // [T*k, H]
    size_t bytes;
};

F32Workspace carve_f32(void* base, int T, int k, int H, int I) {
    F32Workspace w{};
    char* p = static_cast<char*>(base);
    size_t off = 0;
    auto take = [&](size_t n) -> char* {
        char* r = p ? p + off : nullptr;
        off += vmi::align256(n);
        return r;
    };
    const size_t np = (size_t)T * k;
    w.status = reinterpret_cast<uint32_t*>(take(256));
    w.route = reinterpret_cast<RouteInfo*>(take(sizeof(RouteInfo)));
    w.prow = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * np));
    w.act = reinterpret_cast<float*>(take(sizeof(float) * np * I));
    w.y = reinterpret_cast<float*>(take(sizeof(float) * np * H));
    w.bytes = off;
    return w;
}

template <int I>
void launch_down_f32_t(const F32Workspace& ws, vmi_qmat down, int T, int k, int H, hipStream_t s) {
    const dim3 grid(T * k * (H / FRow<I>::RPB));
    hipLaunchKernelGGL((k_down_f32<I>), grid, dim3(kThreads), 0, s, ws.route, down, T, k, H, ws.act, ws.y);
}

template <typename XT>
hipError_t launch_moe_f32(const F32Args& fa, const XT* x, vmi_qmat down, int H, const F32Workspace& ws,
                          void* out, int out_dtype, hipStream_t s) {
    const int T = fa.ra.T, k = fa.ra.k, I = fa.ra.I;
    const dim3 ggrid(T * k * (I / FRow<512>::RPB));
    switch (H) {
        case 512: hipLaunchKernelGGL((k_gateup_f32<512, XT>), ggrid, dim3(kThreads), 0, s, fa, x, ws.act, ws.prow); break;
        case 1024: hipLaunchKernelGGL((k_gateup_f32<1024, XT>), ggrid, dim3(kThreads), 0, s, fa, x, ws.act, ws.prow); break;
        default: hipLaunchKernelGGL((k_gateup_f32<2048, XT>), ggrid, dim3(kThreads), 0, s, fa, x, ws.act, ws.prow); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    switch (I / 64) {
        case 1: launch_down_f32_t<64>(ws, down, T, k, H, s); break;
        case 2: launch_down_f32_t<128>(ws, down, T, k, H, s); break;
        case 3: launch_down_f32_t<192>(ws, down, T, k, H, s); break;
        case 4: launch_down_f32_t<256>(ws, down, T, k, H, s); break;
        case 5: launch_down_f32_t<320>(ws, down, T, k, H, s); break;
        case 6: launch_down_f32_t<384>(ws, down, T, k, H, s); break;
        case 7: launch_down_f32_t<448>(ws, down, T, k, H, s); break;
        default: launch_down_f32_t<512>(ws, down, T, k, H, s); break;
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_combine_f32, dim3((T * H + kThreads - 1) / kThreads), dim3(kThreads), 0, s, ws.prow,
                       fa.ra.in_scores, ws.y, T, k, H, out, out_dtype);
    return hipGetLastError();
}

}  // namespace

namespace vmi {

MoeWorkspace carve_workspace(void* base, int T, int k, int hidden, int inter, int num_experts) {
    MoeWorkspace w{};
    char* p = static_cast<char*>(base);
    size_t off = 0;
    auto take = [&](size_t n) -> char* {
        char* r = p ? p + off : nullptr;
        off += align256(n);
        return r;
    };
    const size_t nrows = (size_t)T * k + T;  // one partial row set per pair, then the shared expert's per token
    w.status = reinterpret_cast<uint32_t*>(take(256));
    w.route = reinterpret_cast<RouteInfo*>(take(sizeof(RouteInfo)));
    w.logits = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T * (num_experts > 0 ? num_experts : 1)));
    w.sg_logit = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.xop = reinterpret_cast<vmi_u4*>(take(sizeof(uint16_t) * (size_t)T * hidden));
    w.xsum = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T * (hidden / 64)));
    w.fscale = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.part = reinterpret_cast<uint16_t*>(take(sizeof(uint16_t) * nrows * (inter / 64) * hidden));
    w.bytes = off;
    return w;
}

}  // namespace vmi

extern "C" size_t vmi_fused_moe_slots_workspace_bytes(int T, int k, int hidden, int inter) {
    if (T <= 0 || k <= 0 || hidden <= 0 || inter <= 0) return 0;
    return carve_f32(nullptr, T, k, hidden, inter).bytes;
}

extern "C" size_t vmi_moe_layer_workspace_bytes(int T, int top_k, int hidden, int inter, int num_experts) {
    if (T <= 0 || top_k <= 0 || hidden <= 0 || inter <= 0 || num_experts <= 0) return 0;
    return vmi::carve_workspace(nullptr, T, top_k, hidden, inter, num_experts).bytes;
}

namespace {

// vmi_fused_moe_slots with a slot list, or vmi_fused_moe_staged without one
// (pair p reads matrix p of stacks holding T*k matrices).
int fused_moe_pairs(const void* x, int x_dtype, bool staged, const int32_t* local_slots, const float* scores,
                    vmi_qmat gate, vmi_qmat up, vmi_qmat down, int T, int k, int hidden, int inter, int group,
                    int bits, int cap, void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                    void* stream) {
    vmi::clear_error();
    int rc = check_shape(T, k, hidden, inter, group, bits);
    if (rc) return rc;
    if (!x || !scores || !out) return vmi::fail(VMI_ERR_INVALID, "null x/scores/out");
    if (!staged && !local_slots) return vmi::fail(VMI_ERR_INVALID, "null local_slots");
    if (x_dtype != VMI_F32 && x_dtype != VMI_BF16) return vmi::fail(VMI_ERR_INVALID, "x_dtype=%d", x_dtype);
    if (out_dtype != VMI_F32 && out_dtype != VMI_BF16) return vmi::fail(VMI_ERR_INVALID, "out_dtype=%d", out_dtype);
    if (!aligned(x, 16)) return vmi::fail(VMI_ERR_INVALID, "x must be 16-byte aligned");
    if (!qmat_ok(gate) || !qmat_ok(up) || !qmat_ok(down))
        return vmi::fail(VMI_ERR_INVALID, "weight arrays must be non-null and 16-byte aligned");
    if (cap <= 0) return vmi::fail(VMI_ERR_INVALID, "cap=%d", cap);
    const size_t need = vmi_fused_moe_slots_workspace_bytes(T, k, hidden, inter);
    if (!workspace || workspace_bytes < need)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", need, workspace_bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // the reference operator's fp32 arithmetic for either x dtype
    const F32Workspace fw = carve_f32(workspace, T, k, hidden, inter);
    F32Args fa{};
    fa.ra.T = T; fa.ra.I = inter; fa.ra.k = k; fa.ra.E = 0; fa.ra.npairs = T * k;
    fa.ra.from_slots = 1; fa.ra.norm = 1; fa.ra.cap = cap;
    fa.ra.slots = local_slots; fa.ra.in_scores = scores;
    fa.ra.route = fw.route; fa.ra.status = fw.status;
    fa.gate = gate; fa.up = up;
    const hipError_t e =
        x_dtype == VMI_F32
            ? launch_moe_f32(fa, static_cast<const float*>(x), down, hidden, fw, out, out_dtype, s)
            : launch_moe_f32(fa, static_cast<const uint16_t*>(x), down, hidden, fw, out, out_dtype, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "fp32 MoE launch");
    return VMI_OK;
}

}  // namespace

extern "C" int vmi_fused_moe_slots(const void* x, int x_dtype, const int32_t* local_slots, const float* scores,
                                   vmi_qmat gate, vmi_qmat up, vmi_qmat down, int T, int k, int hidden, int inter,
                                   int group, int bits, int cap, void* out, int out_dtype, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    return fused_moe_pairs(x, x_dtype, false, local_slots, scores, gate, up, down, T, k, hidden, inter, group, bits, cap, out,
                           out_dtype, workspace, workspace_bytes, stream);
}

extern "C" int vmi_fused_moe_staged(const void* x, int x_dtype, const float* scores, vmi_qmat gate, vmi_qmat up,
                                    vmi_qmat down, int T, int k, int hidden, int inter, int group, int bits,
                                    void* out, int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
    return fused_moe_pairs(x, x_dtype, true, nullptr, scores, gate, up, down, T, k, hidden, inter, group, bits, T * k, out,
                           out_dtype, workspace, workspace_bytes, stream);
}

namespace {

// Argument checks of vmi_moe_layer (and its no-allocation variant); VMI_OK when
// the layer can run.
int check_moe_layer(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* out) {
    if (!desc) return vmi::fail(VMI_ERR_INVALID, "null desc");
    const vmi_moe_layer_desc& D = *desc;
    int rc = check_shape(T, D.top_k, D.hidden, D.inter, D.group, D.bits);
    if (rc) return rc;
    if (D.num_experts <= 0 || D.num_experts > kMaxE || D.num_experts % 64)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "num_experts=%d must be a multiple of 64 up to %d", D.num_experts, kMaxE);
    if (D.top_k > D.num_experts) return vmi::fail(VMI_ERR_INVALID, "top_k > num_experts");
    if (D.router_bits != 4 && D.router_bits != 8) return vmi::fail(VMI_ERR_UNSUPPORTED, "router_bits=%d", D.router_bits);
    const int has_shared = D.shared_gate.w != nullptr;
    const int has_sgate = has_shared && D.shared_expert_gate.w != nullptr;
    if (has_sgate && D.shared_expert_gate_bits != 4 && D.shared_expert_gate_bits != 8)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "shared_expert_gate_bits=%d", D.shared_expert_gate_bits);
    if (!x || !out) return vmi::fail(VMI_ERR_INVALID, "null x/out");
    if (!aligned(x, 16) || !aligned(out, 4)) return vmi::fail(VMI_ERR_INVALID, "x must be 16-byte aligned");
    if (x == out) return vmi::fail(VMI_ERR_INVALID, "out must not alias x");
    if (D.norm_weight && !aligned(D.norm_weight, 16)) return vmi::fail(VMI_ERR_INVALID, "norm_weight alignment");
    if (!qmat_ok(D.router) || !qmat_ok(D.gate) || !qmat_ok(D.up) || !qmat_ok(D.down))
        return vmi::fail(VMI_ERR_INVALID, "router/gate/up/down arrays must be non-null and 16-byte aligned");
    if (has_shared && (!qmat_ok(D.shared_gate) || !qmat_ok(D.shared_up) || !qmat_ok(D.shared_down)))
        return vmi::fail(VMI_ERR_INVALID, "shared expert arrays must be non-null and 16-byte aligned");
    if (has_sgate && !qmat_ok(D.shared_expert_gate)) return vmi::fail(VMI_ERR_INVALID, "shared_expert_gate arrays");
    if (D.cap <= 0) return vmi::fail(VMI_ERR_INVALID, "cap=%d", D.cap);
    return VMI_OK;
}

// The three kernels of one MoE layer call on a carved workspace.
int launch_moe_layer(const vmi_moe_layer_desc& D, const uint16_t* x, int T, const uint16_t* residual, uint16_t* out,
                     int32_t* ids_out, float* scores_out, const vmi::MoeWorkspace& ws, hipStream_t s) {
    const int has_shared = D.shared_gate.w != nullptr;
    const int has_sgate = has_shared && D.shared_expert_gate.w != nullptr;
    const OperandOut ops{ws.xop, ws.xsum, ws.fscale};

    RouterArgs ra{};
    ra.x = x; ra.norm_w = D.norm_weight; ra.eps = D.norm_eps;
    ra.T = T; ra.H = D.hidden; ra.E = D.num_experts;
    ra.router = D.router; ra.rbits = D.router_bits; ra.bias = D.router_logit_bias;
    ra.sgate = has_sgate ? D.shared_expert_gate : D.router;
    ra.sgbits = has_sgate ? D.shared_expert_gate_bits : D.router_bits;
    ra.has_sgate = has_sgate;
    // row groups of 4 waves x kRouterRows rows covering the router rows, the
    // shared-expert gate and one more wave (the one that writes the MFMA
    // operands), times T tokens, in whole blocks of 8 groups (one per XCD)
    constexpr int waves_per_wg = kThreads / VMI_WAVE;
    const int row_waves = (D.num_experts + has_sgate + kRouterRows - 1) / kRouterRows + 1;
    ra.row_wgs = (row_waves + waves_per_wg - 1) / waves_per_wg;
    ra.logits = ws.logits; ra.sg_logit = ws.sg_logit; ra.ops = ops;
    const dim3 rgrid((unsigned)(((ra.row_wgs + 7) / 8) * 8 * T));
    switch (D.hidden) {
        case 512: hipLaunchKernelGGL(k_router<8>, rgrid, dim3(kThreads), 0, s, ra); break;
        case 1024: hipLaunchKernelGGL(k_router<16>, rgrid, dim3(kThreads), 0, s, ra); break;
        default: hipLaunchKernelGGL(k_router<32>, rgrid, dim3(kThreads), 0, s, ra); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_router launch");

    ExpertArgs ea{};
    ea.ra.T = T; ea.ra.I = D.inter; ea.ra.k = D.top_k; ea.ra.E = D.num_experts; ea.ra.npairs = T * D.top_k;
    ea.ra.from_slots = 0; ea.ra.norm = D.norm_topk_prob; ea.ra.cap = D.cap;
    ea.ra.logits = ws.logits; ea.ra.table = D.slot_table;
    ea.ra.route = ws.route; ea.ra.status = ws.status; ea.ra.ids_out = ids_out; ea.ra.scores_out = scores_out;
    ea.has_shared = has_shared; ea.has_sgate = has_sgate;
    ea.gate = D.gate; ea.up = D.up; ea.down = D.down;
    ea.sh_gate = has_shared ? D.shared_gate : D.gate;
    ea.sh_up = has_shared ? D.shared_up : D.up;
    ea.sh_down = has_shared ? D.shared_down : D.down;
    ea.xop = ws.xop; ea.xsum = ws.xsum; ea.fscale = ws.fscale; ea.sg_logit = ws.sg_logit;
    ea.part = ws.part;
    e = launch_experts(ea, D.hidden, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_experts launch");

    CombineArgs ca{};
    ca.T = T; ca.H = D.hidden; ca.NC = D.inter / kSlice; ca.k = D.top_k; ca.npairs = T * D.top_k;
    ca.has_shared = has_shared;
    ca.route = ws.route; ca.part = ws.part; ca.residual = residual; ca.out = out;
    hipLaunchKernelGGL(k_moe_combine, dim3(D.hidden / kCbRows), dim3(kThreads), 0, s, ca);
    e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_moe_combine launch");
    return VMI_OK;
}

// Static scratch of vmi_moe_layer_noalloc: one copy per device, held until the
// process ends.  Host code never passes the array's name to a kernel (on the
// host it is a stand-in, not a device address): every use goes through the
// per-device address from hipGetSymbolAddress.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
constexpr int kMaxDevices = 64;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {nullptr};

// Device address of the current device's scratch, looked up once per device.
int scratch_for_current_device(void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return vmi::hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return vmi::fail(VMI_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return vmi::hip_fail(e, "hipGetSymbolAddress(scratch)");
        if (!p) return vmi::fail(VMI_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return VMI_OK;
}

}  // namespace

extern "C" int vmi_moe_layer(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* residual,
                             uint16_t* out, int32_t* ids_out, float* scores_out, void* workspace,
                             size_t workspace_bytes, void* stream) {
    vmi::clear_error();
    int rc = check_moe_layer(desc, x, T, out);
    if (rc) return rc;
    const vmi_moe_layer_desc& D = *desc;
    const vmi::MoeWorkspace ws = vmi::carve_workspace(workspace, T, D.top_k, D.hidden, D.inter, D.num_experts);
    if (!workspace || workspace_bytes < ws.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", ws.bytes, workspace_bytes);
    return launch_moe_layer(D, x, T, residual, out, ids_out, scores_out, ws, static_cast<hipStream_t>(stream));
}

extern "C" int vmi_moe_layer_noalloc(const vmi_moe_layer_desc* desc, const uint16_t* x, int T,
                                     const uint16_t* residual, uint16_t* out, int32_t* ids_out, float* scores_out,
                                     uint32_t* status, void* stream) {
    vmi::clear_error();
    int rc = check_moe_layer(desc, x, T, out);
    if (rc) return rc;
    const vmi_moe_layer_desc& D = *desc;
    const size_t need = vmi::carve_workspace(nullptr, T, D.top_k, D.hidden, D.inter, D.num_experts).bytes;
    if (need > kNoAllocScratchBytes)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d top_k=%d hidden=%d inter=%d num_experts=%d needs %zu bytes of "
                         "scratch, beyond the static %zu", T, D.top_k, D.hidden, D.inter, D.num_experts, need,
                         kNoAllocScratchBytes);
    void* base = nullptr;
    rc = scratch_for_current_device(&base);
    if (rc) return rc;
    vmi::MoeWorkspace ws = vmi::carve_workspace(base, T, D.top_k, D.hidden, D.inter, D.num_experts);
    // the device status bits go to the caller's word (left as they are when
    // the caller gives none: the scratch's own word is never read)
    if (status) ws.status = status;
    return launch_moe_layer(D, x, T, residual, out, ids_out, scores_out, ws, static_cast<hipStream_t>(stream));
}

#ifdef VMI_TIMELINE
// Tuning builds only: where the kernels of this file record their stamps.
extern "C" int vmi_timeline_set(void* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(vmi_tl_buf), &buf, sizeof(buf)) == hipSuccess ? VMI_OK : VMI_ERR_HIP;
}
#endif

extern "C" int vmi_workspace_status(void* workspace, void* stream, uint32_t* flags) {
    vmi::clear_error();
    if (!workspace || !flags) return vmi::fail(VMI_ERR_INVALID, "null workspace/flags");
    hipStream_t s = static_cast<hipStream_t>(stream);
    uint32_t* dev = static_cast<uint32_t*>(workspace);
    uint32_t host = 0;
    hipError_t e = hipMemcpyAsync(&host, dev, sizeof(uint32_t), hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e == hipSuccess) e = hipMemsetAsync(dev, 0, sizeof(uint32_t), s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return vmi::hip_fail(e, "reading workspace status");
    *flags = host;
    return VMI_OK;
}
