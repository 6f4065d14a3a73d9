// Fused 4-bit MoE for the speculative-decode verify batch (T <= 16 tokens).
//
// Four stream-ordered kernels per layer; kernel boundaries carry every
// cross-workgroup dependency (no fences, no counters, no spin waits):
//   k_router   one wave per router row: every load issued up front, the
//              optional pre-MoE RMSNorm computed from the same registers, the
//              logit in a fixed fp32 order (bit-identical to the CPU oracle).
//              T extra workgroups write the MoE input once in MFMA operand
//              order.
//   k_route    one workgroup: softmax + top-k + renorm per token (DPP wave
//              arg-max over 64-bit rank keys), slot table, distinct slots.
//   k_experts  a fixed grid of workgroups walking the item list (shared-expert
//              slices first, then every distinct slot's 64-row slices of the
//              intermediate dimension): gate and up over the full hidden
//              dimension, SwiGLU, then those 64 activations times the matching
//              64 columns of the down projection for every output row ->
//              per-slice partial outputs.  Every weight load of an item is
//              issued before any arithmetic.  4-bit weights enter the MFMA as
//              exact fp16 subnormals; all tokens routed to a slot share one
//              pass over its weights.
//   k_combine  out = sum_j score_j * sum_slices(partial) + gate * shared
//              (+ residual), fixed summation order.
// vmi_fused_moe_slots runs k_prep (operands + the distinct-slot table of the
// caller's slot list) in place of k_router and k_route.
//
// Semantics follow native/ext/compute/fused_moe.cpp:221-298 (slot pair kernel
// and reduce_pairs) and mlx_streaming/core/moe/block.py:102-109, 321-329, 1008.

#include "vmi_device.h"
#include "vmi_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kExpertWaves = 8;
constexpr int kExpertThreads = kExpertWaves * VMI_WAVE;
constexpr int kMaxT = 16;
constexpr int kMaxPairs = 160;
constexpr int kMaxK = 16;
constexpr int kMaxE = 1024;
constexpr int kSlice = 64;      // intermediate rows per k_experts workgroup
constexpr int kMaxSlices = 8;   // inter <= 512
constexpr float kTwo24 = 16777216.0f;

using vmi::RouteInfo;

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

// bf16 hi/mid/lo split of per-group activation sums as the A operand of the
// bias MFMA: lane block kb = 0, 1, 2 carries hi, mid, lo of groups 0..NG-1.
template <int NG>
__device__ __forceinline__ vmi_u4 make_bias_operand(const float (&X)[NG], int kb) {
    uint16_t p[8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        uint16_t v = 0;
        if (g < NG && kb < 3) {
            const float x = X[g < NG ? g : 0];
            const uint16_t hi = vmi_f32_to_bf16(x);
            const float r1 = x - vmi_bf16_to_f32(hi);
            const uint16_t mid = vmi_f32_to_bf16(r1);
            const uint16_t lo = vmi_f32_to_bf16(r1 - vmi_bf16_to_f32(mid));
            v = kb == 0 ? hi : (kb == 1 ? mid : lo);
        }
        p[g] = v;
    }
    vmi_u4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
    return r;
}

// NG consecutive bf16 values kept packed (NG <= 4): element g in bits 16*(g%2)
// of word g/2.
template <int NG>
__device__ __forceinline__ uint2 load_bf16_packed(const uint16_t* __restrict__ p) {
    if constexpr (NG == 4) {
        return *reinterpret_cast<const uint2*>(p);
    } else if constexpr (NG == 2) {
        return make_uint2(*reinterpret_cast<const uint32_t*>(p), 0u);
    } else {
        return make_uint2((uint32_t)p[0], 0u);
    }
}

__device__ __forceinline__ uint32_t bf16_bits_at(const uint2& v, int g) {
    const uint32_t w = (g >> 1) ? v.y : v.x;
    return (g & 1) ? (w >> 16) : (w & 0xffffu);
}

// B operand of the bias MFMA: lane blocks kb < 3 carry the row's NG biases.
template <int NG>
__device__ __forceinline__ vmi_u4 bias_b_operand(const uint2& bb, int kb) {
    vmi_u4 r = {0u, 0u, 0u, 0u};
    if (kb < 3) {
        r[0] = bb.x;
        r[1] = bb.y;
    }
    return r;
}

// Raw loads of one 16-row x NG-group tile of a 4-bit projection (lane row
// l%16, k block l/16).
template <int NG>
struct TileLoad {
    uint2 w[NG];
    uint2 s, b;
};

// Buffer-load form: wr/sr/br cover one expert's matrix / scales / biases, woff
// and soff are the lane's byte offsets of its row (+ k block) and the block's
// uniform offsets are added as scalar offsets.
template <int NG>
__device__ __forceinline__ void tile_load_rsrc(TileLoad<NG>& tl, __amdgpu_buffer_rsrc_t wr, __amdgpu_buffer_rsrc_t sr,
                                               __amdgpu_buffer_rsrc_t br, uint32_t woff, uint32_t sboff,
                                               uint32_t w_uni, uint32_t sb_uni) {
#pragma unroll
    for (int g = 0; g < NG; ++g) tl.w[g] = vmi_bload_b64(wr, woff, w_uni + 32u * g);
    if constexpr (NG == 4) {
        tl.s = vmi_bload_b64(sr, sboff, sb_uni);
        tl.b = vmi_bload_b64(br, sboff, sb_uni);
    } else if constexpr (NG == 2) {
        tl.s = make_uint2(vmi_bload_b32(sr, sboff, sb_uni), 0u);
        tl.b = make_uint2(vmi_bload_b32(br, sboff, sb_uni), 0u);
    } else {
        tl.s = make_uint2(vmi_bload_b16(sr, sboff, sb_uni), 0u);
        tl.b = make_uint2(vmi_bload_b16(br, sboff, sb_uni), 0u);
    }
}

// D[token][row] (activation-scaled units) of a loaded tile against the
// activation operands ax (per group, two MFMA halves) and bias operand aX.
template <int NG>
__device__ __forceinline__ vmi_f4 tile_mma(const TileLoad<NG>& tl, const vmi_u4 (&ax)[NG][2], const vmi_u4& aX,
                                           int kb) {
    const vmi_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    vmi_f4 acc = zero;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        vmi_f4 m = vmi_mfma_f16(ax[g][0], vmi_unpack_u4_f16(tl.w[g].x), zero);
        m = vmi_mfma_f16(ax[g][1], vmi_unpack_u4_f16(tl.w[g].y), m);
        const float sc = vmi_bf16_to_f32(bf16_bits_at(tl.s, g));
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = fmaf(sc, m[r], acc[r]);
    }
    const vmi_f4 accb = vmi_mfma_bf16(aX, bias_b_operand<NG>(tl.b, kb), zero);
    vmi_f4 d;
#pragma unroll
    for (int r = 0; r < 4; ++r) d[r] = fmaf(acc[r], kTwo24, accb[r]);
    return d;
}

template <typename XT>
__device__ __forceinline__ void load_x8(const XT* __restrict__ row, int c, float (&v)[8]);

template <>
__device__ __forceinline__ void load_x8<uint16_t>(const uint16_t* __restrict__ row, int c, float (&v)[8]) {
    unpack_bf16x8(*reinterpret_cast<const uint4*>(row + c), v);
}

template <>
__device__ __forceinline__ void load_x8<float>(const float* __restrict__ row, int c, float (&v)[8]) {
    const float4 p = *reinterpret_cast<const float4*>(row + c);
    const float4 q = *reinterpret_cast<const float4*>(row + c + 4);
    v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
    v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
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
    vmi_u4* xop;    // [T, H/64, 4, 2] MFMA operands
    float* xsum;    // [T, H/64]
    float* fscale;  // [T]
};

// One 256-thread workgroup writes the MFMA operands of token t: the MoE input
// (x, or the RMSNorm output rounded to bf16) scaled by a power of two f with
// max|x f| in (2^13, 2^14], in fp16, per-group sums, and f.
template <typename XT, int CPL>
__device__ void write_operands(const XT* __restrict__ xrow, const uint16_t* __restrict__ norm_w, float eps, int H,
                               int t, const OperandOut& o) {
    __shared__ float s_red[kThreads / VMI_WAVE];
    __shared__ float s_inv;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    constexpr int kChunksPerThread = (64 * CPL) / (8 * kThreads) > 0 ? (64 * CPL) / (8 * kThreads) : 1;
    const bool active = 8 * tid < H;
    float v[kChunksPerThread][8];
#pragma unroll
    for (int ch = 0; ch < kChunksPerThread; ++ch) {
        const int c0 = 8 * tid + ch * 8 * kThreads;
        if (active) {
            load_x8<XT>(xrow, c0, v[ch]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[ch][i] = 0.0f;
        }
    }
    float inv = 1.0f;
    if (norm_w) {
        if constexpr (sizeof(XT) == 2) {
            if (w == 0) {
                uint4 xr[CPL / 8];
#pragma unroll
                for (int ch = 0; ch < CPL / 8; ++ch)
                    xr[ch] = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(xrow) + lane * CPL +
                                                             8 * ch);
                const float iv = canonical_inv_rms<CPL / 8>(xr, H, eps);
                if (lane == 0) s_inv = iv;
            }
        }
        __syncthreads();
        inv = s_inv;
#pragma unroll
        for (int ch = 0; ch < kChunksPerThread; ++ch) {
            if (active) {
                float nw[8];
                load_x8<uint16_t>(norm_w, 8 * tid + ch * 8 * kThreads, nw);
#pragma unroll
                for (int i = 0; i < 8; ++i) v[ch][i] = vmi_bf16r((v[ch][i] * inv) * nw[i]);
            }
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int ch = 0; ch < kChunksPerThread; ++ch)
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[ch][i]));
    amax = vmi_wave_max(amax);
    if (lane == 0) s_red[w] = amax;
    __syncthreads();
    float am = s_red[0];
#pragma unroll
    for (int i = 1; i < kThreads / VMI_WAVE; ++i) am = fmaxf(am, s_red[i]);
    const float f = vmi_fp16_range_scale(am);
    const int G = H / 64;
#pragma unroll
    for (int ch = 0; ch < kChunksPerThread; ++ch) {
        const int c0 = 8 * tid + ch * 8 * kThreads;
        float xs = 0.0f;
        const vmi_u4 op = make_act_operand(v[ch], f, xs);
        // group sum over the 8 threads holding one 64-column group
        xs += __shfl_xor(xs, 1, VMI_WAVE);
        xs += __shfl_xor(xs, 2, VMI_WAVE);
        xs += __shfl_xor(xs, 4, VMI_WAVE);
        if (active) {
            const int g = c0 / 64, kb = (c0 % 64) / 16, m = (c0 % 16) / 8;
            o.xop[(((size_t)t * G + g) * 4 + kb) * 2 + m] = op;
            if ((tid & 7) == 0) o.xsum[(size_t)t * G + g] = xs;
        }
    }
    if (tid == 0) o.fscale[t] = f;
}

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
    int row_wgs;      // workgroups carrying router rows
    float* logits;    // [T, E]
    float* sg_logit;  // [T]
    OperandOut ops;
};

// Router rows: one wave per row (plus one for the shared-expert gate).  Lane l
// owns columns [l*CPL, (l+1)*CPL), accumulating fmaf(w, x, acc) in column
// order; the 64 partials meet in the canonical wave-sum tree.  The CPU oracle reproduces
// this order bit for bit (orc_router_logits_f32).  Workgroups past row_wgs
// each write one token's MFMA operands.
template <int CPL>
__global__ __launch_bounds__(kThreads) void k_router(RouterArgs a) {
    constexpr int NCH = CPL / 8;  // packed 8-column chunks per lane
    constexpr int TB = 4;         // tokens per register batch
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int T = a.T, H = a.H;
    if ((int)blockIdx.x >= a.row_wgs) {
        const int t = blockIdx.x - a.row_wgs;
        write_operands<uint16_t, CPL>(a.x + (size_t)t * H, a.norm_w, a.eps, H, t, a.ops);
        return;
    }
    const int row = blockIdx.x * (kThreads / VMI_WAVE) + w;
    if (row >= a.E + a.has_sgate) return;
    const bool is_sg = row >= a.E;
    const vmi_qmat m = is_sg ? a.sgate : a.router;
    const int bits = is_sg ? a.sgbits : a.rbits;
    const int r = is_sg ? 0 : row;
    const int G = H / 64;
    const int c0 = lane * CPL;
    // weights: 8-bit -> CPL/4 words, 4-bit -> CPL/8 words of this lane's columns
    uint32_t wword[CPL / 4];
    const uint32_t* wrow = m.w + (size_t)r * (size_t)(H * bits / 32) + (size_t)c0 * bits / 32;
#pragma unroll
    for (int i = 0; i < CPL / 4; ++i) wword[i] = (bits == 8 || i < CPL / 8) ? wrow[i] : 0u;
    // scales/biases of the groups the lane's columns touch
    constexpr int NGL = CPL >= 64 ? CPL / 64 : 1;
    uint16_t sv[NGL], bv[NGL];
#pragma unroll
    for (int i = 0; i < NGL; ++i) {
        sv[i] = m.s[(size_t)r * G + c0 / 64 + i];
        bv[i] = m.b[(size_t)r * G + c0 / 64 + i];
    }
    uint4 nwv[NCH];
    if (a.norm_w) {
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) nwv[ch] = *reinterpret_cast<const uint4*>(a.norm_w + c0 + 8 * ch);
    }
    for (int tb = 0; tb < T; tb += TB) {
        uint4 xr[TB][NCH];
#pragma unroll
        for (int q = 0; q < TB; ++q)
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch)
                xr[q][ch] = (tb + q < T) ? *reinterpret_cast<const uint4*>(a.x + (size_t)(tb + q) * H + c0 + 8 * ch)
                                         : make_uint4(0u, 0u, 0u, 0u);
        float inv[TB];
#pragma unroll
        for (int q = 0; q < TB; ++q) inv[q] = a.norm_w ? canonical_inv_rms<NCH>(xr[q], H, a.eps) : 1.0f;
        float acc[TB];
#pragma unroll
        for (int q = 0; q < TB; ++q) acc[q] = 0.0f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            const int gi = (8 * ch) / 64;
            const float sc = vmi_bf16_to_f32(sv[gi < NGL ? gi : 0]);
            const float bi = vmi_bf16_to_f32(bv[gi < NGL ? gi : 0]);
            float wv[8];
            if (bits == 4) {
                const uint32_t word = wword[ch];
#pragma unroll
                for (int i = 0; i < 8; ++i) wv[i] = fmaf((float)((word >> (4 * i)) & 15u), sc, bi);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[i] = fmaf((float)((wword[2 * ch] >> (8 * i)) & 255u), sc, bi);
#pragma unroll
                for (int i = 0; i < 4; ++i) wv[4 + i] = fmaf((float)((wword[2 * ch + 1] >> (8 * i)) & 255u), sc, bi);
            }
            float nw[8];
            if (a.norm_w) unpack_bf16x8(nwv[ch], nw);
#pragma unroll
            for (int q = 0; q < TB; ++q) {
                float xf[8];
                unpack_bf16x8(xr[q][ch], xf);
                if (a.norm_w) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) xf[i] = vmi_bf16r((xf[i] * inv[q]) * nw[i]);
                }
                float s = acc[q];
#pragma unroll
                for (int i = 0; i < 8; ++i) s = fmaf(wv[i], xf[i], s);
                acc[q] = s;
            }
        }
#pragma unroll
        for (int q = 0; q < TB; ++q) {
            float v = vmi_wave_sum_canon(acc[q]);
            if (lane == 0 && tb + q < T) {
                if (is_sg) {
                    a.sg_logit[tb + q] = v;
                } else {
                    if (a.bias) v = v + a.bias[row];
                    a.logits[(size_t)(tb + q) * a.E + row] = v;
                }
            }
        }
    }
}

// ----------------------------------------------------------- routing
// Routing state of one verify batch while it is being built, in LDS.
struct RouteLds {
    int32_t ids[kMaxPairs];
    float scores[kMaxPairs];
    int32_t slot[kMaxPairs];
    int32_t rank[kMaxPairs];
    int32_t uidx[kMaxPairs];
    int32_t psrc[kMaxPairs];
    int32_t uslot[kMaxPairs];
    uint32_t umask[kMaxPairs];
    int32_t wcnt[kThreads / VMI_WAVE];
    int32_t U;
    uint32_t bad;
};

constexpr int kFirstTable = 4096;  // LDS first-occurrence table covers cap <= 4096

// Softmax + top-k + renorm of token t's logits by one wave (block.py:321-329):
// k rounds of a wave-wide maximum over 64-bit rank keys (value descending,
// lower expert index first, NaN last).  Writes the token's k pairs to LDS.
__device__ void topk_token(const float* __restrict__ lt, int E, int k, int norm, int t, RouteLds& R) {
    const int lane = threadIdx.x & 63;
    const int NI = E / 64;
    float v[kMaxE / 64];
    uint64_t key[kMaxE / 64];
#pragma unroll
    for (int i = 0; i < kMaxE / 64; ++i) {
        v[i] = (i < NI) ? lt[lane + 64 * i] : 0.0f;
        key[i] = (i < NI) ? vmi_rank_key(v[i], lane + 64 * i) : 0ull;
    }
    float sel_val[kMaxK];
    int sel_idx[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        sel_val[j] = 0.0f;
        sel_idx[j] = 0;
        if (j < k) {
            uint64_t best = 0ull;
#pragma unroll
            for (int i = 0; i < kMaxE / 64; ++i) best = vmi_u64_max(best, key[i]);
            const uint64_t win = vmi_wave_max_u64(best);
            const int idx = (int)(0xffffffffu - (uint32_t)win);
            sel_idx[j] = idx;
            sel_val[j] = vmi_order_key_value((uint32_t)(win >> 32));
#pragma unroll
            for (int i = 0; i < kMaxE / 64; ++i)
                if (key[i] == win) key[i] = 0ull;  // taken (keys are unique per index)
        }
    }
    const float mx = sel_val[0];
    bool bad = false;
    float e[kMaxK];
    float den = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        e[j] = 0.0f;
        if (j < k) {
            bad |= !(fabsf(sel_val[j]) < 3.0e38f);
            e[j] = expf(sel_val[j] - mx);
            if (norm) den = den + e[j];
        }
    }
    if (!norm) {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxE / 64; ++i)
            if (i < NI) part = part + expf(v[i] - mx);
        den = vmi_wave_sum_canon(part);
    }
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (j < k && lane == j) {
            R.ids[t * k + j] = sel_idx[j];
            R.scores[t * k + j] = e[j] / den;
        }
    }
    if (bad && lane == 0) atomicOr(&R.bad, VMI_STATUS_BAD_ROUTE);
}

// Distinct valid slots in first-appearance order over the token-major pair
// list (R.slot filled, -1 = invalid; cap <= kFirstTable uses an LDS
// first-occurrence table).  Fills rank/uidx/psrc/uslot/umask/U.  Called by all
// threads of a 256-thread workgroup.
__device__ void dedup_lds(int npairs, int k, int cap, RouteLds& R, int32_t* s_first) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const bool table = cap <= kFirstTable;
    if (tid < kMaxPairs) R.umask[tid] = 0u;
    if (table)
        for (int i = tid; i < cap; i += kThreads) s_first[i] = 0x7fffffff;
    __syncthreads();
    if (table && tid < npairs && R.slot[tid] >= 0) atomicMin(&s_first[R.slot[tid]], tid);
    __syncthreads();
    bool first = false;
    int fidx = -1;
    if (tid < npairs) {
        const int s = R.slot[tid];
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
            first = (fidx == tid);
        }
    }
    const uint64_t bal = __ballot(first);
    if (lane == 0) R.wcnt[w] = __popcll(bal);
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += R.wcnt[i];
    const int rank = base + __popcll(bal & ((1ull << lane) - 1ull));
    if (first) {
        R.rank[tid] = rank;
        R.uslot[rank] = R.slot[tid];
    }
    __syncthreads();
    if (tid < npairs) {
        const int u = fidx >= 0 ? R.rank[fidx] : -1;
        const int t = tid / k;
        int src = -1;
        if (u >= 0) {
            atomicOr(&R.umask[u], 1u << t);
            src = tid;
            for (int q = t * k; q < tid; ++q) {
                if (R.slot[q] == R.slot[tid]) {
                    src = q;
                    break;
                }
            }
        }
        R.uidx[tid] = u;
        R.psrc[tid] = src;
    }
    if (tid == 0) {
        int U = 0;
        for (int i = 0; i < kThreads / VMI_WAVE; ++i) U += R.wcnt[i];
        R.U = U;
    }
    __syncthreads();
}

// RouteLds -> RouteInfo in global memory (all threads).
__device__ void publish_route(int npairs, int k, const RouteLds& R, RouteInfo* ri) {
    const int tid = threadIdx.x;
    for (int i = tid; i < kMaxPairs * kMaxT; i += kThreads) (&ri->upair[0][0])[i] = -1;
    __syncthreads();
    if (tid < npairs) {
        ri->uslot[tid] = R.uslot[tid];
        ri->umask[tid] = R.umask[tid];
        ri->psrc[tid] = R.psrc[tid];
        if (R.psrc[tid] == tid) ri->upair[R.uidx[tid]][tid / k] = (int16_t)tid;
    }
    if (tid == 0) ri->U = R.U;
}

struct RouteArgs {
    int T, E, k, norm, cap;
    const float* logits;   // [T, E]
    const float* sg_logit; // [T] or nullptr
    const int32_t* table;  // [E] or nullptr
    float* sg;
    float* scores;         // [T*k]
    RouteInfo* route;
    uint32_t* status;
    int32_t* ids_out;
    float* scores_out;
};

// One workgroup: wave w ranks tokens w, w+4, ...; then slots and the
// distinct-slot table.
__global__ __launch_bounds__(kThreads) void k_route(RouteArgs a) {
    __shared__ RouteLds R;
    __shared__ int32_t s_table[kMaxE];
    __shared__ int32_t s_first[kFirstTable];
    const int tid = threadIdx.x, w = tid >> 6;
    const int T = a.T, npairs = T * a.k;
    if (a.table)
        for (int e = tid; e < a.E; e += kThreads) s_table[e] = a.table[e];
    if (tid == 0) R.bad = 0u;
    __syncthreads();
    for (int t = w; t < T; t += kThreads / VMI_WAVE) topk_token(a.logits + (size_t)t * a.E, a.E, a.k, a.norm, t, R);
    __syncthreads();
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
    dedup_lds(npairs, a.k, a.cap, R, s_first);
    publish_route(npairs, a.k, R, a.route);
    if (tid < npairs) {
        a.scores[tid] = R.scores[tid];
        if (a.ids_out) a.ids_out[tid] = R.ids[tid];
        if (a.scores_out) a.scores_out[tid] = R.scores[tid];
    }
    if (tid < T && a.sg_logit) a.sg[tid] = 1.0f / (1.0f + expf(-a.sg_logit[tid]));
    if (tid == 0 && R.bad) atomicOr(a.status, R.bad);
}

// --------------------------------------------------------------- prep (slots API)
struct PrepArgs {
    const void* x;
    int T, H, k, cap;
    const int32_t* slots;
    RouteInfo* route;
    uint32_t* status;
    OperandOut ops;
};

// Workgroups 0..T-1 write operands; workgroup T writes the distinct-slot
// table of the caller's slots.
template <typename XT, int CPL>
__global__ __launch_bounds__(kThreads) void k_prep(PrepArgs a) {
    __shared__ RouteLds R;
    __shared__ int32_t s_first[kFirstTable];
    if ((int)blockIdx.x < a.T) {
        const int t = blockIdx.x;
        write_operands<XT, CPL>(reinterpret_cast<const XT*>(a.x) + (size_t)t * a.H, nullptr, 0.0f, a.H, t, a.ops);
        return;
    }
    const int tid = threadIdx.x;
    const int npairs = a.T * a.k;
    if (tid < npairs) {
        const int s = a.slots[tid];
        const bool ok = s >= 0 && s < a.cap;
        R.slot[tid] = ok ? s : -1;
        if (!ok) atomicOr(a.status, VMI_STATUS_BAD_SLOT);
    }
    __syncthreads();
    dedup_lds(npairs, a.k, a.cap, R, s_first);
    publish_route(npairs, a.k, R, a.route);
}

// ---------------------------------------------------------------- experts
struct ExpertArgs {
    int T, H, I, npairs, has_shared;
    const RouteInfo* route;
    vmi_qmat gate, up, down, sh_gate, sh_up, sh_down;
    const vmi_u4* xop;
    const float* xsum;
    const float* fscale;
    float* part;  // [npairs + T, I/64, H]; routed pair p or npairs + t for the shared expert
};

// One workgroup (8 waves) per item i = blockIdx.x (the grid covers the most
// items a batch can have; workgroups past the batch's count exit at once):
// items [0, NC) are the shared expert's slices (when present), then distinct
// slot u's slices c at has_shared*NC + u*NC + c, so the shared expert is
// dispatched first.  Per item:
// phase 1: wave w takes hidden groups [GW*w, GW*w+GW) of the four 16-row
// blocks of gate and up (k split), partials meet in LDS in fixed wave order;
// phase 2: the slice's 64 activations (one quantisation group of the down
// projection) times down column group c for all H output rows.
template <int GW>
__global__ __launch_bounds__(kExpertThreads, 1) void k_experts(ExpertArgs a) {
    __shared__ float s_red[kExpertWaves][2][4][VMI_WAVE];
    __shared__ float s_act[kMaxT][kSlice + 1];
    __shared__ float s_fa[kMaxT];
    __shared__ float s_xa[kMaxT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int i16 = lane & 15, kb = lane >> 4;
    const int T = a.T, H = a.H, I = a.I;
    const int NC = I / kSlice;
    const int G = H / 64;
    const int G0 = w * GW;
    const int H8 = H / 8, I8 = I / 8, GI = I / 64;
    const int ntile = H / 16;
    const int nsh = a.has_shared ? NC : 0;
    const int U = a.route->U;
    const int nitems = nsh + U * NC;
    const bool tok_ok = i16 < T;
    // reduction-thread token (tid < 256): t = 4*(l2/16) + r
    const int red_t = 4 * ((tid & 63) >> 4) + (tid >> 6);
    const float red_inv = (tid < 256 && red_t < T) ? 1.0f / a.fscale[red_t] : 0.0f;

    {
        const int item = blockIdx.x;
        if (item >= nitems) return;
        const bool is_shared = item < nsh;
        const int u = is_shared ? -1 : (item - nsh) / NC;
        const int c = is_shared ? item : (item - nsh) % NC;
        const int slot = is_shared ? 0 : a.route->uslot[u];
        const uint32_t tmask = is_shared ? ((T >= 32) ? 0xffffffffu : ((1u << T) - 1u)) : a.route->umask[u];
        int prow[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 4 * kb + r;
            prow[r] = (t < T) ? (is_shared ? a.npairs + t : (int)a.route->upair[u][t]) : -1;
        }
        const vmi_qmat mg = is_shared ? a.sh_gate : a.gate;
        const vmi_qmat mu = is_shared ? a.sh_up : a.up;
        const vmi_qmat md = is_shared ? a.sh_down : a.down;

        // every weight load of the item first: phase 1 (gate/up) then phase 2 (down),
        // through buffer resources over this expert's matrices (uniform bases,
        // one lane offset each, per-tile offsets in scalar registers)
        const __amdgpu_buffer_rsrc_t rgw = vmi_rsrc(mg.w + (size_t)slot * I * H8, (uint32_t)I * H8 * 4u);
        const __amdgpu_buffer_rsrc_t rgs = vmi_rsrc(mg.s + (size_t)slot * I * G, (uint32_t)I * G * 2u);
        const __amdgpu_buffer_rsrc_t rgb = vmi_rsrc(mg.b + (size_t)slot * I * G, (uint32_t)I * G * 2u);
        const __amdgpu_buffer_rsrc_t ruw = vmi_rsrc(mu.w + (size_t)slot * I * H8, (uint32_t)I * H8 * 4u);
        const __amdgpu_buffer_rsrc_t rus = vmi_rsrc(mu.s + (size_t)slot * I * G, (uint32_t)I * G * 2u);
        const __amdgpu_buffer_rsrc_t rub = vmi_rsrc(mu.b + (size_t)slot * I * G, (uint32_t)I * G * 2u);
        const uint32_t row1 = (uint32_t)(c * kSlice + i16);
        const uint32_t woff1 = (row1 * H8 + 8u * G0 + 2u * kb) * 4u;
        const uint32_t sboff1 = (row1 * G + G0) * 2u;
        TileLoad<GW> lg[4], lu[4];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            const uint32_t wu = (uint32_t)(blk * 16 * H8 * 4), su = (uint32_t)(blk * 16 * G * 2);
            tile_load_rsrc<GW>(lg[blk], rgw, rgs, rgb, woff1, sboff1, wu, su);
            tile_load_rsrc<GW>(lu[blk], ruw, rus, rub, woff1, sboff1, wu, su);
        }
        constexpr int kTilesPerWave = 2048 / 16 / kExpertWaves;  // H <= 2048
        const __amdgpu_buffer_rsrc_t rdw = vmi_rsrc(md.w + (size_t)slot * H * I8, (uint32_t)H * I8 * 4u);
        const __amdgpu_buffer_rsrc_t rds = vmi_rsrc(md.s + (size_t)slot * H * GI, (uint32_t)H * GI * 2u);
        const __amdgpu_buffer_rsrc_t rdb = vmi_rsrc(md.b + (size_t)slot * H * GI, (uint32_t)H * GI * 2u);
        const uint32_t row2 = (uint32_t)(w * 16 + i16);
        const uint32_t woff2 = (row2 * I8 + 8u * c + 2u * kb) * 4u;
        const uint32_t sboff2 = (row2 * GI + c) * 2u;
        uint2 dw[kTilesPerWave];
        uint32_t ds[kTilesPerWave], db[kTilesPerWave];
        // tile j = w + 8i covers rows 16*j + i16 = row2 + 128*i; the first half
        // goes out with phase 1, the second after the phase-1 MFMAs
        auto load_down = [&](int i) {
            const uint32_t rowu = (uint32_t)(kExpertWaves * 16 * i);
            dw[i] = vmi_bload_b64(rdw, woff2, rowu * I8 * 4u);
            ds[i] = vmi_bload_b16(rds, sboff2, rowu * GI * 2u);
            db[i] = vmi_bload_b16(rdb, sboff2, rowu * GI * 2u);
        };

        // activation operands of token i16 for this wave's groups
        vmi_u4 ax[GW][2];
        float X[GW];
#pragma unroll
        for (int g = 0; g < GW; ++g) {
            if (tok_ok) {
                const size_t base = (((size_t)i16 * G + G0 + g) * 4 + kb) * 2;
                ax[g][0] = a.xop[base];
                ax[g][1] = a.xop[base + 1];
                X[g] = a.xsum[(size_t)i16 * G + G0 + g];
            } else {
                ax[g][0] = ax[g][1] = vmi_u4{0u, 0u, 0u, 0u};
                X[g] = 0.0f;
            }
        }
        const vmi_u4 aX = make_bias_operand<GW>(X, kb);
        // consume phase-1 tiles in load order; each half of the down loads is
        // issued once two blocks' registers are free (compiler barriers keep
        // the order: loads return in issue order)
        vmi_f4 dg[4], du[4];
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            dg[blk] = tile_mma<GW>(lg[blk], ax, aX, kb);
            du[blk] = tile_mma<GW>(lu[blk], ax, aX, kb);
            if (blk == 1 || blk == 3) {
                asm volatile("" ::: "memory");
                const int i0 = blk == 1 ? 0 : kTilesPerWave / 2;
#pragma unroll
                for (int i = 0; i < kTilesPerWave / 2; ++i) load_down(i0 + i);
                asm volatile("" ::: "memory");
            }
        }
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            __syncthreads();  // the previous reduction (or item) has finished with s_red / s_act
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                s_red[w][0][r][lane] = dg[blk][r];
                s_red[w][1][r][lane] = du[blk][r];
            }
            __syncthreads();
            if (tid < 256 && red_t < T) {
                const int l2 = tid & 63, r = tid >> 6;
                float g = 0.0f, up = 0.0f;
#pragma unroll
                for (int ww = 0; ww < kExpertWaves; ++ww) {
                    g += s_red[ww][0][r][l2];
                    up += s_red[ww][1][r][l2];
                }
                g *= red_inv;
                up *= red_inv;
                s_act[red_t][blk * 16 + (l2 & 15)] =
                    ((tmask >> red_t) & 1u) ? g * (1.0f / (1.0f + expf(-g))) * up : 0.0f;
            }
        }
        __syncthreads();
        if (w == 0) {
            // per-token range factor over the 64 activations (lanes = columns)
            for (int t = 0; t < T; ++t) {
                const float am = vmi_wave_max(fabsf(s_act[t][lane]));
                if (lane == 0) s_fa[t] = vmi_fp16_range_scale(am);
            }
        }
        __syncthreads();
        // down operand of token i16: columns 16*kb + 8*m + perm[s]
        vmi_u4 aa[2];
        float xa = 0.0f;
        const float fa = tok_ok ? s_fa[i16] : 1.0f;
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = tok_ok ? s_act[i16][16 * kb + 8 * m + i] : 0.0f;
            aa[m] = make_act_operand(v, fa, xa);
        }
        xa += __shfl_xor(xa, 16, VMI_WAVE);
        xa += __shfl_xor(xa, 32, VMI_WAVE);
        if (w == 0 && kb == 0 && tok_ok) s_xa[i16] = xa;
        __syncthreads();
        float xat[4], ifa[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 4 * kb + r;
            xat[r] = (t < T) ? s_xa[t] : 0.0f;
            ifa[r] = (t < T) ? 1.0f / s_fa[t] : 0.0f;
        }
        const vmi_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < kTilesPerWave; ++i) {
            const int j = w + kExpertWaves * i;
            if (j < ntile) {
                vmi_f4 mm = vmi_mfma_f16(aa[0], vmi_unpack_u4_f16(dw[i].x), zero);
                mm = vmi_mfma_f16(aa[1], vmi_unpack_u4_f16(dw[i].y), mm);
                const float sc = vmi_bf16_to_f32(ds[i]) * kTwo24;
                const float bi = vmi_bf16_to_f32(db[i]);
                const int row = j * 16 + i16;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (prow[r] >= 0)
                        a.part[((size_t)prow[r] * NC + c) * H + row] = fmaf(sc, mm[r], bi * xat[r]) * ifa[r];
                }
            }
        }
    }
}

// ---------------------------------------------------------------- combine
struct CombineArgs {
    int T, H, k, npairs, has_shared;
    const RouteInfo* route;
    const float* scores;
    const float* sg;
    const float* part;
    const uint16_t* residual;
    void* out;
    int out_dtype;
};

// out[t][h] = sum_j scores[t,j] * (sum over slices, ascending) + gate_t *
// shared (+ residual), all in fp32 in fixed order.  Every load is issued
// before the first use.
template <int NC>
__global__ __launch_bounds__(kThreads) void k_combine(CombineArgs a) {
    const int idx = blockIdx.x * kThreads + threadIdx.x;
    if (idx >= a.T * a.H) return;
    const int t = idx / a.H, h = idx - t * a.H;
    const size_t pstride = (size_t)NC * a.H;
    int src[kMaxK];
    float sc[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        src[j] = (j < a.k) ? a.route->psrc[t * a.k + j] : -1;
        sc[j] = (j < a.k) ? a.scores[t * a.k + j] : 0.0f;
    }
    float y[kMaxK + 1][NC];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j)
#pragma unroll
        for (int c = 0; c < NC; ++c) y[j][c] = (src[j] >= 0) ? a.part[(size_t)src[j] * pstride + (size_t)c * a.H + h] : 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
        y[kMaxK][c] = a.has_shared ? a.part[(size_t)(a.npairs + t) * pstride + (size_t)c * a.H + h] : 0.0f;
    const float gsh = (a.has_shared && a.sg) ? a.sg[t] : 1.0f;
    const float res = a.residual ? vmi_bf16_to_f32(a.residual[idx]) : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        if (src[j] >= 0) {
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < NC; ++c) s += y[j][c];
            acc = fmaf(sc[j], s, acc);
        }
    }
    if (a.has_shared) {
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) s += y[kMaxK][c];
        acc = fmaf(gsh, s, acc);
    }
    if (a.residual) acc += res;
    if (a.out_dtype == VMI_BF16)
        reinterpret_cast<uint16_t*>(a.out)[idx] = vmi_f32_to_bf16(acc);
    else
        reinterpret_cast<float*>(a.out)[idx] = acc;
}

// ---------------------------------------------------------------- host
bool aligned(const void* p, size_t n) { return ((uintptr_t)p % n) == 0; }

bool qmat_ok(const vmi_qmat& m) { return m.w && m.s && m.b && aligned(m.w, 8) && aligned(m.s, 8) && aligned(m.b, 8); }

int check_shape(int T, int k, int hidden, int inter, int group, int bits) {
    if (T <= 0 || k <= 0) return vmi::fail(VMI_ERR_INVALID, "T=%d and k=%d must be positive", T, k);
    if (T > kMaxT) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d exceeds %d (verify batch limit)", T, kMaxT);
    if (T * k > kMaxPairs) return vmi::fail(VMI_ERR_UNSUPPORTED, "T*k=%d exceeds %d", T * k, kMaxPairs);
    if (k > kMaxK) return vmi::fail(VMI_ERR_UNSUPPORTED, "k=%d exceeds %d", k, kMaxK);
    if (bits != 4 || group != 64)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "only bits=4, group=64 is built (got bits=%d group=%d)", bits, group);
    if (hidden != 512 && hidden != 1024 && hidden != 2048)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d not in {512,1024,2048}", hidden);
    if (inter % kSlice || inter < kSlice || inter > kSlice * kMaxSlices)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "inter=%d must be a multiple of 64 up to %d", inter, kSlice * kMaxSlices);
    return VMI_OK;
}

hipError_t launch_experts(const ExpertArgs& ea, hipStream_t s) {
    const dim3 grid((ea.npairs + ea.has_shared) * (ea.I / kSlice));
    switch (ea.H) {
        case 512: hipLaunchKernelGGL((k_experts<1>), grid, dim3(kExpertThreads), 0, s, ea); break;
        case 1024: hipLaunchKernelGGL((k_experts<2>), grid, dim3(kExpertThreads), 0, s, ea); break;
        default: hipLaunchKernelGGL((k_experts<4>), grid, dim3(kExpertThreads), 0, s, ea); break;
    }
    return hipGetLastError();
}

hipError_t launch_combine(const CombineArgs& ca, int nslice, hipStream_t s) {
    const dim3 grid((ca.T * ca.H + kThreads - 1) / kThreads);
    switch (nslice) {
        case 1: hipLaunchKernelGGL(k_combine<1>, grid, dim3(kThreads), 0, s, ca); break;
        case 2: hipLaunchKernelGGL(k_combine<2>, grid, dim3(kThreads), 0, s, ca); break;
        case 3: hipLaunchKernelGGL(k_combine<3>, grid, dim3(kThreads), 0, s, ca); break;
        case 4: hipLaunchKernelGGL(k_combine<4>, grid, dim3(kThreads), 0, s, ca); break;
        case 5: hipLaunchKernelGGL(k_combine<5>, grid, dim3(kThreads), 0, s, ca); break;
        case 6: hipLaunchKernelGGL(k_combine<6>, grid, dim3(kThreads), 0, s, ca); break;
        case 7: hipLaunchKernelGGL(k_combine<7>, grid, dim3(kThreads), 0, s, ca); break;
        default: hipLaunchKernelGGL(k_combine<8>, grid, dim3(kThreads), 0, s, ca); break;
    }
    return hipGetLastError();
}

template <typename XT>
void launch_prep(const PrepArgs& pa, hipStream_t s) {
    const dim3 grid(pa.T + 1);
    switch (pa.H) {
        case 512: hipLaunchKernelGGL((k_prep<XT, 8>), grid, dim3(kThreads), 0, s, pa); break;
        case 1024: hipLaunchKernelGGL((k_prep<XT, 16>), grid, dim3(kThreads), 0, s, pa); break;
        default: hipLaunchKernelGGL((k_prep<XT, 32>), grid, dim3(kThreads), 0, s, pa); break;
    }
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
    const size_t npairs = (size_t)T * k;
    w.status = reinterpret_cast<uint32_t*>(take(256));
    w.route = reinterpret_cast<RouteInfo*>(take(sizeof(RouteInfo)));
    w.logits = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T * (num_experts > 0 ? num_experts : 1)));
    w.sg_logit = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.sg = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.ids = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * npairs));
    w.scores = reinterpret_cast<float*>(take(sizeof(float) * npairs));
    w.slots = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * npairs));
    w.xop = reinterpret_cast<vmi_u4*>(take(sizeof(uint16_t) * (size_t)T * hidden));
    w.xsum = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T * (hidden / 64)));
    w.fscale = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.part = reinterpret_cast<float*>(take(sizeof(float) * (npairs + T) * (size_t)(inter / 64) * hidden));
    w.bytes = off;
    return w;
}

}  // namespace vmi

extern "C" size_t vmi_fused_moe_slots_workspace_bytes(int T, int k, int hidden, int inter) {
    if (T <= 0 || k <= 0 || hidden <= 0 || inter <= 0) return 0;
    return vmi::carve_workspace(nullptr, T, k, hidden, inter, 0).bytes;
}

extern "C" size_t vmi_moe_layer_workspace_bytes(int T, int top_k, int hidden, int inter, int num_experts) {
    if (T <= 0 || top_k <= 0 || hidden <= 0 || inter <= 0 || num_experts <= 0) return 0;
    return vmi::carve_workspace(nullptr, T, top_k, hidden, inter, num_experts).bytes;
}

extern "C" int vmi_fused_moe_slots(const void* x, int x_dtype, const int32_t* local_slots, const float* scores,
                                   vmi_qmat gate, vmi_qmat up, vmi_qmat down, int T, int k, int hidden, int inter,
                                   int group, int bits, int cap, void* out, int out_dtype, void* workspace,
                                   size_t workspace_bytes, void* stream) {
    vmi::clear_error();
    int rc = check_shape(T, k, hidden, inter, group, bits);
    if (rc) return rc;
    if (!x || !local_slots || !scores || !out) return vmi::fail(VMI_ERR_INVALID, "null x/local_slots/scores/out");
    if (x_dtype != VMI_F32 && x_dtype != VMI_BF16) return vmi::fail(VMI_ERR_INVALID, "x_dtype=%d", x_dtype);
    if (out_dtype != VMI_F32 && out_dtype != VMI_BF16) return vmi::fail(VMI_ERR_INVALID, "out_dtype=%d", out_dtype);
    if (!aligned(x, 16)) return vmi::fail(VMI_ERR_INVALID, "x must be 16-byte aligned");
    if (!qmat_ok(gate) || !qmat_ok(up) || !qmat_ok(down))
        return vmi::fail(VMI_ERR_INVALID, "weight arrays must be non-null and 8-byte aligned");
    if (cap <= 0) return vmi::fail(VMI_ERR_INVALID, "cap=%d", cap);
    const vmi::MoeWorkspace ws = vmi::carve_workspace(workspace, T, k, hidden, inter, 0);
    if (!workspace || workspace_bytes < ws.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", ws.bytes, workspace_bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const OperandOut ops{ws.xop, ws.xsum, ws.fscale};

    const PrepArgs pa{x, T, hidden, k, cap, local_slots, ws.route, ws.status, ops};
    if (x_dtype == VMI_BF16)
        launch_prep<uint16_t>(pa, s);
    else
        launch_prep<float>(pa, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_prep launch");

    ExpertArgs ea{};
    ea.T = T; ea.H = hidden; ea.I = inter; ea.npairs = T * k; ea.has_shared = 0;
    ea.route = ws.route;
    ea.gate = gate; ea.up = up; ea.down = down; ea.sh_gate = gate; ea.sh_up = up; ea.sh_down = down;
    ea.xop = ws.xop; ea.xsum = ws.xsum; ea.fscale = ws.fscale; ea.part = ws.part;
    e = launch_experts(ea, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_experts launch");

    CombineArgs ca{};
    ca.T = T; ca.H = hidden; ca.k = k; ca.npairs = T * k; ca.has_shared = 0;
    ca.route = ws.route; ca.scores = scores; ca.sg = nullptr; ca.part = ws.part;
    ca.residual = nullptr; ca.out = out; ca.out_dtype = out_dtype;
    e = launch_combine(ca, inter / kSlice, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_combine launch");
    return VMI_OK;
}

extern "C" int vmi_moe_layer(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* residual,
                             uint16_t* out, int32_t* ids_out, float* scores_out, void* workspace,
                             size_t workspace_bytes, void* stream) {
    vmi::clear_error();
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
        return vmi::fail(VMI_ERR_INVALID, "router/gate/up/down arrays must be non-null and aligned");
    if (has_shared && (!qmat_ok(D.shared_gate) || !qmat_ok(D.shared_up) || !qmat_ok(D.shared_down)))
        return vmi::fail(VMI_ERR_INVALID, "shared expert arrays must be non-null and aligned");
    if (has_sgate && !qmat_ok(D.shared_expert_gate)) return vmi::fail(VMI_ERR_INVALID, "shared_expert_gate arrays");
    if (D.cap <= 0) return vmi::fail(VMI_ERR_INVALID, "cap=%d", D.cap);
    const vmi::MoeWorkspace ws = vmi::carve_workspace(workspace, T, D.top_k, D.hidden, D.inter, D.num_experts);
    if (!workspace || workspace_bytes < ws.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", ws.bytes, workspace_bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const OperandOut ops{ws.xop, ws.xsum, ws.fscale};

    RouterArgs ra{};
    ra.x = x; ra.norm_w = D.norm_weight; ra.eps = D.norm_eps;
    ra.T = T; ra.H = D.hidden; ra.E = D.num_experts;
    ra.router = D.router; ra.rbits = D.router_bits; ra.bias = D.router_logit_bias;
    ra.sgate = has_sgate ? D.shared_expert_gate : D.router;
    ra.sgbits = has_sgate ? D.shared_expert_gate_bits : D.router_bits;
    ra.has_sgate = has_sgate;
    ra.row_wgs = (D.num_experts + has_sgate + 3) / 4;
    ra.logits = ws.logits; ra.sg_logit = ws.sg_logit; ra.ops = ops;
    const dim3 rgrid(ra.row_wgs + T);
    switch (D.hidden) {
        case 512: hipLaunchKernelGGL(k_router<8>, rgrid, dim3(kThreads), 0, s, ra); break;
        case 1024: hipLaunchKernelGGL(k_router<16>, rgrid, dim3(kThreads), 0, s, ra); break;
        default: hipLaunchKernelGGL(k_router<32>, rgrid, dim3(kThreads), 0, s, ra); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_router launch");

    RouteArgs ta{};
    ta.T = T; ta.E = D.num_experts; ta.k = D.top_k; ta.norm = D.norm_topk_prob; ta.cap = D.cap;
    ta.logits = ws.logits; ta.sg_logit = has_sgate ? ws.sg_logit : nullptr; ta.table = D.slot_table;
    ta.sg = ws.sg; ta.scores = ws.scores; ta.route = ws.route; ta.status = ws.status;
    ta.ids_out = ids_out; ta.scores_out = scores_out;
    hipLaunchKernelGGL(k_route, dim3(1), dim3(kThreads), 0, s, ta);
    e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_route launch");

    ExpertArgs ea{};
    ea.T = T; ea.H = D.hidden; ea.I = D.inter; ea.npairs = T * D.top_k; ea.has_shared = has_shared;
    ea.route = ws.route;
    ea.gate = D.gate; ea.up = D.up; ea.down = D.down;
    ea.sh_gate = has_shared ? D.shared_gate : D.gate;
    ea.sh_up = has_shared ? D.shared_up : D.up;
    ea.sh_down = has_shared ? D.shared_down : D.down;
    ea.xop = ws.xop; ea.xsum = ws.xsum; ea.fscale = ws.fscale; ea.part = ws.part;
    e = launch_experts(ea, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_experts launch");

    CombineArgs ca{};
    ca.T = T; ca.H = D.hidden; ca.k = D.top_k; ca.npairs = T * D.top_k; ca.has_shared = has_shared;
    ca.route = ws.route; ca.scores = ws.scores; ca.sg = has_sgate ? ws.sg : nullptr; ca.part = ws.part;
    ca.residual = residual; ca.out = out; ca.out_dtype = VMI_BF16;
    e = launch_combine(ca, D.inter / kSlice, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_combine launch");
    return VMI_OK;
}

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
