// Fused 4-bit MoE for the speculative-decode verify batch (T <= 16 tokens).
//
// Three stream-ordered kernels per layer; kernel boundaries carry every
// cross-workgroup dependency (no fences, no counters, no spin waits):
//   k_router    router logits, one wave per two router rows: the optional
//               pre-MoE RMSNorm is computed once per workgroup into LDS, the
//               logit accumulates in a fixed fp32 order (bit-identical to the
//               CPU oracle).  T extra workgroups write the MoE input once in
//               MFMA operand order.
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
//   k_downcomb  one workgroup per 16 output rows: every distinct slot's down
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

#include "vmi_device.h"
#include "vmi_internal.h"

namespace {

constexpr int kThreads = 256;
constexpr int kDownWaves = 8;
constexpr int kDownThreads = kDownWaves * VMI_WAVE;
constexpr int kMaxT = 16;
constexpr int kMaxPairs = 160;
constexpr int kMaxK = 16;
constexpr int kMaxE = 1024;
constexpr int kSlice = 64;        // intermediate rows per k_gateup workgroup (= one down group)
constexpr int kMaxInter = 512;
constexpr int kFirstTable = 1024; // LDS first-occurrence table covers cap <= 1024
constexpr int kTPad = 16;         // token stride of the per-group inverse range factors
constexpr float kTwo24 = 16777216.0f;

static_assert(kMaxPairs == vmi::kRouteMaxPairs && kMaxT == vmi::kRouteMaxT, "route table sizes");

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

// Affine-bias term sum_g b[row][g] * X[t][g] as one bf16 MFMA: X is split into
// bf16 hi + mid + lo (24 significant bits); lane block q carries two groups:
//   A = [hi(X0), mid(X0), lo(X0), 0, hi(X1), mid(X1), lo(X1), 0]
//   B = [b0, b0, b0, 0, b1, b1, b1, 0]   (b0/b1 = low/high bf16 of one word)
__device__ __forceinline__ void split3_bf16(float x, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
    hi = vmi_f32_to_bf16(x);
    const float r1 = x - vmi_bf16_to_f32(hi);
    mid = vmi_f32_to_bf16(r1);
    lo = vmi_f32_to_bf16(r1 - vmi_bf16_to_f32(mid));
}
__device__ __forceinline__ vmi_u4 bias_a_operand(float x0, float x1) {
    uint32_t h0, m0, l0, h1, m1, l1;
    split3_bf16(x0, h0, m0, l0);
    split3_bf16(x1, h1, m1, l1);
    vmi_u4 r;
    r[0] = h0 | (m0 << 16);
    r[1] = l0;
    r[2] = h1 | (m1 << 16);
    r[3] = l1;
    return r;
}
__device__ __forceinline__ vmi_u4 bias_b_operand(uint32_t bb) {
    const uint32_t b0 = bb & 0xffffu, b1 = bb >> 16;
    vmi_u4 r;
    r[0] = b0 | (b0 << 16);
    r[1] = b0;
    r[2] = b1 | (b1 << 16);
    r[3] = b1;
    return r;
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
    vmi_u4* xop;    // [T, H/8] MFMA operands
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
            o.xop[(size_t)t * (H / 8) + c0 / 8] = op;
            if ((tid & 7) == 0) o.xsum[(size_t)t * G + c0 / 64] = xs;
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

constexpr int kRouterRowsPerWave = 2;

// Router rows: wave w of workgroup b takes rows 2(4b + w) and 2(4b + w) + 1
// (row E is the shared-expert gate).  Lane l owns columns [l*CPL, (l+1)*CPL),
// accumulating fmaf(w, x, acc) in column order; the 64 partials meet in the
// canonical wave-sum tree.  The (normalised) input is built once per
// workgroup in LDS: wave w normalises tokens w, w+4, ...  The CPU oracle
// reproduces this order bit for bit (orc_router_logits_f32).  Workgroups past
// row_wgs each write one token's MFMA operands.
template <int CPL>
__global__ __launch_bounds__(kThreads) void k_router(RouterArgs a) {
    constexpr int NCH = CPL / 8;  // packed 8-column chunks per lane
    constexpr int RPW = kRouterRowsPerWave;
    __shared__ uint4 s_xn[kMaxT][64 * NCH];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int T = a.T, H = a.H;
    if ((int)blockIdx.x >= a.row_wgs) {
        const int t = blockIdx.x - a.row_wgs;
        write_operands<uint16_t, CPL>(a.x + (size_t)t * H, a.norm_w, a.eps, H, t, a.ops);
        return;
    }
    const int G = H / 64;
    const int c0 = lane * CPL;
    const int row0 = (blockIdx.x * (kThreads / VMI_WAVE) + w) * RPW;
    const int nrows = a.E + a.has_sgate;
    const bool is_sg = row0 >= a.E;  // E is even: a wave holds router rows only or the gate row only
    const vmi_qmat m = is_sg ? a.sgate : a.router;
    const int bits = is_sg ? a.sgbits : a.rbits;
    // weights: 8-bit -> CPL/4 words, 4-bit -> CPL/8 words of this lane's columns
    uint32_t wword[RPW][CPL / 4];
    uint16_t sv[RPW], bv[RPW];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const int row = row0 + k;
        const bool ok = row < nrows;
        const int r = ok ? (is_sg ? 0 : row) : 0;
        const uint32_t* wrow = m.w + (size_t)r * (size_t)(H * bits / 32) + (size_t)c0 * bits / 32;
#pragma unroll
        for (int i = 0; i < CPL / 4; ++i) wword[k][i] = (ok && (bits == 8 || i < CPL / 8)) ? wrow[i] : 0u;
        sv[k] = ok ? m.s[(size_t)r * G + c0 / 64] : (uint16_t)0;
        bv[k] = ok ? m.b[(size_t)r * G + c0 / 64] : (uint16_t)0;
    }
    // the MoE input, normalised, for every token into LDS
    for (int t = w; t < T; t += kThreads / VMI_WAVE) {
        uint4 xr[NCH];
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) xr[ch] = *reinterpret_cast<const uint4*>(a.x + (size_t)t * H + c0 + 8 * ch);
        if (a.norm_w) {
            const float inv = canonical_inv_rms<NCH>(xr, H, a.eps);
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) {
                float xf[8], nw[8];
                unpack_bf16x8(xr[ch], xf);
                unpack_bf16x8(*reinterpret_cast<const uint4*>(a.norm_w + c0 + 8 * ch), nw);
                uint32_t pk[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    pk[i] = (uint32_t)vmi_f32_to_bf16((xf[2 * i] * inv) * nw[2 * i]) |
                            ((uint32_t)vmi_f32_to_bf16((xf[2 * i + 1] * inv) * nw[2 * i + 1]) << 16);
                xr[ch] = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            }
        }
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) s_xn[t][lane * NCH + ch] = xr[ch];
    }
    __syncthreads();
    if (row0 >= nrows) return;
    // dequantised weights (w = q*s + b is exact in fp32)
    float wv[RPW][CPL];
#pragma unroll
    for (int k = 0; k < RPW; ++k) {
        const float sc = vmi_bf16_to_f32(sv[k]), bi = vmi_bf16_to_f32(bv[k]);
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const uint32_t qv = (bits == 4) ? (wword[k][c / 8] >> (4 * (c % 8))) & 15u
                                            : (wword[k][c / 4] >> (8 * (c % 4))) & 255u;
            wv[k][c] = fmaf((float)qv, sc, bi);
        }
    }
    for (int t = 0; t < T; ++t) {
        // chunk reads rotated by lane/4 (4 chunks) or lane/8 (2 chunks) to spread LDS banks
        uint4 xr[NCH];
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int ch = (NCH == 1) ? 0 : ((i + (NCH == 4 ? (lane >> 2) : (lane >> 3))) & (NCH - 1));
            const uint4 v = s_xn[t][lane * NCH + ch];
#pragma unroll
            for (int cc = 0; cc < NCH; ++cc)
                if (cc == ch) xr[cc] = v;
        }
        float acc[RPW];
#pragma unroll
        for (int k = 0; k < RPW; ++k) acc[k] = 0.0f;
#pragma unroll
        for (int ch = 0; ch < NCH; ++ch) {
            float xf[8];
            unpack_bf16x8(xr[ch], xf);
#pragma unroll
            for (int k = 0; k < RPW; ++k)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[k] = fmaf(wv[k][8 * ch + i], xf[i], acc[k]);
        }
#pragma unroll
        for (int k = 0; k < RPW; ++k) {
            float v = vmi_wave_sum_canon(acc[k]);
            const int row = row0 + k;
            if (lane == 0 && row < nrows) {
                if (is_sg) {
                    a.sg_logit[t] = v;
                } else {
                    if (a.bias) v = v + a.bias[row];
                    a.logits[(size_t)t * a.E + row] = v;
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
    int32_t slot[kMaxPairs];   // -1 = invalid
    int32_t rank[kMaxPairs];   // distinct index, stored at first-occurrence pairs
    int32_t uslot[kMaxPairs];
    uint32_t umask[kMaxPairs];
    int32_t wcnt[kThreads / VMI_WAVE];
    int32_t U;
    uint32_t bad;
};

// Top-k key: larger value first; NaN maps to 1 (below every number), 0 marks
// a taken element.
__device__ __forceinline__ uint32_t topk_key(float f) { return (f != f) ? 1u : vmi_order_key(f); }

// Softmax + top-k + renorm of token t's logits by one wave (block.py:321-329):
// k rounds of a wave-wide maximum over 32-bit value keys; the winner is the
// lowest expert index holding the maximum (ballots in index order).  Writes
// the token's k pairs to LDS.
__device__ void topk_token(const float* __restrict__ lt, int E, int k, int norm, int t, RouteLds& R) {
    const int lane = threadIdx.x & 63;
    const int NI = E / 64;
    float v[kMaxE / 64];
    uint32_t key[kMaxE / 64];
#pragma unroll
    for (int i = 0; i < kMaxE / 64; ++i) {
        v[i] = (i < NI) ? lt[lane + 64 * i] : 0.0f;
        key[i] = (i < NI) ? topk_key(v[i]) : 0u;
    }
    float sel_val[kMaxK];
    int sel_idx[kMaxK];
#pragma unroll
    for (int j = 0; j < kMaxK; ++j) {
        sel_val[j] = 0.0f;
        sel_idx[j] = 0;
        if (j < k) {
            uint32_t mx = key[0];
#pragma unroll
            for (int i = 1; i < kMaxE / 64; ++i) mx = max(mx, key[i]);
            const uint32_t M = vmi_wave_max_u32(mx);
            int idx = -1;
#pragma unroll
            for (int i = 0; i < kMaxE / 64; ++i) {
                if (i < NI && idx < 0) {
                    const uint64_t b = __ballot(key[i] == M);
                    if (b) idx = 64 * i + __builtin_ctzll(b);
                }
            }
#pragma unroll
            for (int i = 0; i < kMaxE / 64; ++i)
                if (64 * i + lane == idx) key[i] = 0u;
            sel_idx[j] = idx;
            sel_val[j] = vmi_order_key_value(M);
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
// list (R.slot filled, -1 = invalid).  cap <= kFirstTable uses an LDS
// first-occurrence table (only the entries of slots in use are touched).
// Fills rank/uslot/umask/U.  Called by all threads of a 256-thread workgroup.
__device__ void dedup_lds(int npairs, int k, int cap, RouteLds& R, int32_t* s_first) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
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

// ---------------------------------------------------------------- gate/up
struct GateUpArgs {
    int T, I, k, E, npairs, has_shared;
    int from_slots;               // 1: caller slots + scores, 0: route from logits
    int norm, cap;
    const float* logits;          // [T, E]
    const int32_t* table;         // [E] or nullptr
    const int32_t* slots;         // [T*k] (from_slots)
    const float* in_scores;       // [T*k] (from_slots)
    vmi_qmat gate, up, sh_gate, sh_up;
    const vmi_u4* xop;            // [T, H/8]
    const float* xsum;            // [T, H/64]
    const float* fscale;          // [T]
    RouteInfo* route;             // written by the first routed workgroup
    uint32_t* status;
    int32_t* ids_out;             // [T*k] or nullptr
    float* scores_out;            // [T*k] or nullptr
    vmi_u4* actop;                // [npairs+1, T, I/8]
    float* axs;                   // [npairs+1, T, I/64]
    float* aifa;                  // [npairs+1, I/64, kTPad]
};

// Routing of the batch inside one k_gateup workgroup (all threads).  The
// workgroup `publish` additionally writes the route table for k_downcomb, the
// caller's ids/scores and the status bits.
__device__ void route_batch(const GateUpArgs& a, RouteLds& R, int32_t* s_table, int32_t* s_first, bool publish) {
    const int tid = threadIdx.x, w = tid >> 6;
    const int T = a.T, k = a.k, npairs = a.npairs;
    if (tid == 0) R.bad = 0u;
    if (!a.from_slots) {
        if (a.table)
            for (int e = tid; e < a.E; e += kThreads) s_table[e] = a.table[e];
        __syncthreads();
        for (int t = w; t < T; t += kThreads / VMI_WAVE)
            topk_token(a.logits + (size_t)t * a.E, a.E, k, a.norm, t, R);
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
    } else {
        __syncthreads();
        if (tid < npairs) {
            const int s = a.slots[tid];
            const bool ok = s >= 0 && s < a.cap;
            R.slot[tid] = ok ? s : -1;
            R.scores[tid] = a.in_scores[tid];
            if (!ok) atomicOr(&R.bad, VMI_STATUS_BAD_SLOT);
        }
    }
    __syncthreads();
    dedup_lds(npairs, k, a.cap, R, s_first);
    if (!publish) return;
    const int U = R.U;
    if (tid == 0) a.route->U = U;
    if (tid < U) a.route->uslot[tid] = R.uslot[tid];
    // combine weight of (u, t): its pairs' scores in j order
    for (int i = tid; i < U * T; i += kThreads) {
        const int u = i / T, t = i - u * T;
        const int s = R.uslot[u];
        float wsum = 0.0f;
        for (int j = 0; j < k; ++j)
            if (R.slot[t * k + j] == s) wsum += R.scores[t * k + j];
        a.route->wt[u][t] = wsum;
    }
    if (tid < npairs && !a.from_slots) {
        if (a.ids_out) a.ids_out[tid] = R.ids[tid];
        if (a.scores_out) a.scores_out[tid] = R.scores[tid];
    }
    if (tid == 0 && R.bad) atomicOr(a.status, R.bad);
}

// One workgroup (4 waves) per item = blockIdx.x: items [0, NC) are the shared
// expert's slices (when present), then distinct slot u's slices c at
// nsh + u*NC + c.  Workgroups past the batch's item count exit after routing.
// Wave w: rows c*64 + 16w + (lane % 16) of gate and up; lane block q = lane/16
// loads 16 bytes at 64m + 16q of its row for m = 0..NM-1 (two groups per m).
template <int NM, bool PACK>
__global__ __launch_bounds__(kThreads, 2) void k_gateup(GateUpArgs a) {
    constexpr int kT = PACK ? 8 : 16;
    constexpr int H = NM * 128, H8 = H / 8, NG = H / 64;
    constexpr int NB = NM / 4;      // bias MFMAs of 8 groups each
    constexpr int NSV = NG / 8;     // 16-byte loads of one row's scales
    constexpr int XPT = (kT * H8 + kThreads - 1) / kThreads;
    __shared__ vmi_u4 s_x[kT][H8 + 1];
    __shared__ float s_xs[kT][NG];
    __shared__ float s_inv[kT];
    __shared__ float s_act[kT][kSlice + 1];
    __shared__ RouteLds R;
    __shared__ int32_t s_table[kMaxE];
    __shared__ int32_t s_first[kFirstTable];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int T = a.T, I = a.I, NC = I / kSlice;
    const int nsh = a.has_shared ? NC : 0;
    const int item = blockIdx.x;
    const bool is_shared = item < nsh;
    const vmi_u4 zero4 = {0u, 0u, 0u, 0u};

    // the MoE input operands go to registers first (they arrive during routing)
    vmi_u4 xr[XPT];
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
        const int idx = tid + kThreads * i;
        xr[i] = (idx < T * H8) ? a.xop[idx] : zero4;
    }
    // (every global load the arithmetic needs is issued before the weight loads:
    // loads retire in issue order)
    constexpr int XSPT = (kT * NG + kThreads - 1) / kThreads;
    float xsr[XSPT];
#pragma unroll
    for (int i = 0; i < XSPT; ++i) {
        const int idx = tid + kThreads * i;
        xsr[i] = (idx < T * NG) ? a.xsum[idx] : 0.0f;
    }
    const float invr = (tid < T) ? 1.0f / a.fscale[tid] : 0.0f;

    int slot = 0, c = item, aidx = a.npairs;
    uint32_t tmask = (1u << T) - 1u;
    if (!is_shared) {
        route_batch(a, R, s_table, s_first, item == nsh);
        const int ii = item - nsh, u = ii / NC;
        if (u >= R.U) return;
        c = ii - u * NC;
        slot = R.uslot[u];
        tmask = R.umask[u];
        aidx = u;
    }

    // every weight load of the item: scales, biases, then gate/up words by m
    const vmi_qmat mg = is_shared ? a.sh_gate : a.gate;
    const vmi_qmat mu = is_shared ? a.sh_up : a.up;
    const uint32_t wbytes = (uint32_t)I * (H / 2), sbytes = (uint32_t)I * NG * 2u;
    const __amdgpu_buffer_rsrc_t rgw = vmi_rsrc(mg.w + (size_t)slot * I * H8, wbytes);
    const __amdgpu_buffer_rsrc_t ruw = vmi_rsrc(mu.w + (size_t)slot * I * H8, wbytes);
    const __amdgpu_buffer_rsrc_t rgs = vmi_rsrc(mg.s + (size_t)slot * I * NG, sbytes);
    const __amdgpu_buffer_rsrc_t rus = vmi_rsrc(mu.s + (size_t)slot * I * NG, sbytes);
    const __amdgpu_buffer_rsrc_t rgb = vmi_rsrc(mg.b + (size_t)slot * I * NG, sbytes);
    const __amdgpu_buffer_rsrc_t rub = vmi_rsrc(mu.b + (size_t)slot * I * NG, sbytes);
    const uint32_t row = (uint32_t)(c * kSlice + 16 * w + r);
    const uint32_t sboff = row * NG * 2u;
    vmi_u4 sg4[NSV], su4[NSV];
#pragma unroll
    for (int i = 0; i < NSV; ++i) {
        sg4[i] = vmi_bload_b128(rgs, sboff, 16u * i);
        su4[i] = vmi_bload_b128(rus, sboff, 16u * i);
    }
    uint32_t bgw[NB], buw[NB];
    {
        const uint32_t boff = sboff + 4u * NB * q;
        if constexpr (NB == 4) {
            const vmi_u4 g = vmi_bload_b128(rgb, boff, 0), u = vmi_bload_b128(rub, boff, 0);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                bgw[b] = g[b];
                buw[b] = u[b];
            }
        } else if constexpr (NB == 2) {
            const uint2 g = vmi_bload_b64(rgb, boff, 0), u = vmi_bload_b64(rub, boff, 0);
            bgw[0] = g.x; bgw[1] = g.y;
            buw[0] = u.x; buw[1] = u.y;
        } else {
            bgw[0] = vmi_bload_b32(rgb, boff, 0);
            buw[0] = vmi_bload_b32(rub, boff, 0);
        }
    }
    const uint32_t woff = row * (uint32_t)(H / 2) + 16u * q;
    vmi_u4 wg[NM], wu[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        wg[m] = vmi_bload_b128(rgw, woff, 64u * m);
        wu[m] = vmi_bload_b128(ruw, woff, 64u * m);
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
        if (idx < T * NG) s_xs[idx / NG][idx % NG] = xsr[i];
    }
    if (tid < T) s_inv[tid] = invr;
    __syncthreads();

    // main MFMAs: m-th load pair covers groups 2m (K blocks 0-1) and 2m+1 (2-3)
    const int par = lane >> 5;  // PACK: D rows 8..15 (lanes 32..63) hold the odd group
    float accg[4] = {0.0f, 0.0f, 0.0f, 0.0f}, accu[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const vmi_f4 zf = {0.0f, 0.0f, 0.0f, 0.0f};
    const int tk = PACK ? (r & 7) : r;
    const bool xreal = PACK ? (((q < 2) == (r < 8)) && tk < T) : (r < T);
    const int tkc = tk < T ? tk : 0;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        vmi_u4 ax[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const vmi_u4 v = s_x[tkc][16 * m + 4 * q + j];
            ax[j] = xreal ? v : zero4;
        }
        const uint32_t swg = sg4[m / 4][m % 4], swu = su4[m / 4][m % 4];
        if constexpr (PACK) {
            vmi_f4 dg = zf, du = zf;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dg = vmi_mfma_f16(ax[j], vmi_unpack_u4_f16(wg[m][j]), dg);
                du = vmi_mfma_f16(ax[j], vmi_unpack_u4_f16(wu[m][j]), du);
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
                const vmi_u4 bg = vmi_unpack_u4_f16(wg[m][j]), bu = vmi_unpack_u4_f16(wu[m][j]);
                dg0 = vmi_mfma_f16(a0, bg, dg0);
                dg1 = vmi_mfma_f16(a1, bg, dg1);
                du0 = vmi_mfma_f16(a0, bu, du0);
                du1 = vmi_mfma_f16(a1, bu, du1);
            }
            const float sg0 = __uint_as_float(swg << 16), sg1 = __uint_as_float(swg & 0xffff0000u);
            const float su0 = __uint_as_float(swu << 16), su1 = __uint_as_float(swu & 0xffff0000u);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                accg[e] = fmaf(sg1, dg1[e], fmaf(sg0, dg0[e], accg[e]));
                accu[e] = fmaf(su1, du1[e], fmaf(su0, du0[e], accu[e]));
            }
        }
    }
    // affine-bias term: lane block q carries groups 2*NB*q + 2b, +1
    vmi_f4 bgd = zf, bud = zf;
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int g0 = 2 * NB * q + 2 * b;
        const vmi_u4 ab = (r < T) ? bias_a_operand(s_xs[r][g0], s_xs[r][g0 + 1]) : zero4;
        bgd = vmi_mfma_bf16(ab, bias_b_operand(bgw[b]), bgd);
        bud = vmi_mfma_bf16(ab, bias_b_operand(buw[b]), bud);
    }
    // SwiGLU of token t = 4*(lane/16) + e, row 16w + r of the slice
    const int tq = lane >> 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        float tg = accg[e], tu = accu[e];
        if constexpr (PACK) {
            tg += __shfl_xor(tg, 32, VMI_WAVE);
            tu += __shfl_xor(tu, 32, VMI_WAVE);
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
    // down-projection operands of this slice: thread (t, kk) packs columns 8kk..8kk+7
    const int NGd = NC;
    if (w < (T + 7) / 8) {
        const int t = 8 * w + (lane >> 3), kk = lane & 7;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (t < T) ? s_act[t][8 * kk + i] : 0.0f;
        float am = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
        am = fmaxf(am, __shfl_xor(am, 1, VMI_WAVE));
        am = fmaxf(am, __shfl_xor(am, 2, VMI_WAVE));
        am = fmaxf(am, __shfl_xor(am, 4, VMI_WAVE));
        const float fa = vmi_fp16_range_scale(am);
        float xs = 0.0f;
        const vmi_u4 op = make_act_operand(v, fa, xs);
        xs += __shfl_xor(xs, 1, VMI_WAVE);
        xs += __shfl_xor(xs, 2, VMI_WAVE);
        xs += __shfl_xor(xs, 4, VMI_WAVE);
        if (t < T) {
            const float ifa = 1.0f / fa;
            a.actop[((size_t)aidx * T + t) * (I / 8) + 8 * c + kk] = op;
            if (kk == 0) {
                a.axs[((size_t)aidx * T + t) * NGd + c] = xs * ifa;
                a.aifa[((size_t)aidx * NGd + c) * kTPad + t] = ifa;
            }
        }
    }
}

// --------------------------------------------------------- down + combine
struct DownArgs {
    int T, H, I, npairs, has_shared, has_sgate;
    const RouteInfo* route;
    vmi_qmat down, sh_down;
    const vmi_u4* actop;
    const float* axs;
    const float* aifa;
    const float* sg_logit;     // [T] (has_sgate)
    const uint16_t* residual;  // [T, H] or nullptr
    void* out;
    int out_dtype;
};

// One workgroup (8 waves) per 16 output rows h0..h0+15.  Wave w takes experts
// e = w, w+8, ... of the list [shared (when present), distinct slots 0..U-1]:
// the 16 down rows x inter of expert e (16-byte loads, two groups per load),
// the expert's activation operands, then weight * (down . act) summed per
// token into registers; the 8 waves' sums meet in LDS in wave order, plus the
// residual.
template <int NMD, bool PACK>
__global__ __launch_bounds__(kDownThreads, 1) void k_downcomb(DownArgs a) {
    __shared__ float s_red[kDownWaves][4][VMI_WAVE];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int q = lane >> 4, r = lane & 15;
    const int T = a.T, H = a.H, I = a.I, I8 = I / 8, NGd = I / 64;
    const int h = blockIdx.x * 16 + r;
    const int tq = lane >> 4;
    const int par = PACK ? (tq >> 1) : 0;
    const int tt0 = PACK ? 4 * (tq & 1) : 4 * tq;  // first token of this lane's D rows
    const vmi_u4 zero4 = {0u, 0u, 0u, 0u};
    const vmi_f4 zf = {0.0f, 0.0f, 0.0f, 0.0f};
    const int tk = PACK ? (r & 7) : r;
    const bool areal = PACK ? (((q < 2) == (r < 8)) && tk < T) : (r < T);
    const int ne = a.has_shared + a.route->U;
    float wsum[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int e = w; e < ne; e += kDownWaves) {
        const bool sh = a.has_shared && e == 0;
        const int u = e - a.has_shared;
        const int aidx = sh ? a.npairs : u;
        const int slot = sh ? 0 : a.route->uslot[u];
        const vmi_qmat md = sh ? a.sh_down : a.down;
        // activation-side operands (L2 resident) before the weights
        const __amdgpu_buffer_rsrc_t ra = vmi_rsrc(a.actop + (size_t)aidx * T * I8, (uint32_t)T * I8 * 16u);
        vmi_u4 A[NMD][4];
#pragma unroll
        for (int m = 0; m < NMD; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int wi = 16 * m + 4 * q + j;
                A[m][j] = vmi_bload_b128(ra, (areal && wi < I8) ? (uint32_t)(tk * I8 + wi) * 16u : VMI_OOB, 0);
            }
        const float* ifa_base = a.aifa + (size_t)aidx * NGd * kTPad;
        float4 ifa0[NMD], ifa1[NMD];
#pragma unroll
        for (int m = 0; m < NMD; ++m) {
            const int g0 = 2 * m + par;
            ifa0[m] = g0 < NGd ? *reinterpret_cast<const float4*>(ifa_base + g0 * kTPad + tt0)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (!PACK) {
                const int g1 = 2 * m + 1;
                ifa1[m] = g1 < NGd ? *reinterpret_cast<const float4*>(ifa_base + g1 * kTPad + tt0)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
        float x0 = 0.0f, x1 = 0.0f;
        if (r < T) {
            const float* xb = a.axs + ((size_t)aidx * T + r) * NGd;
            if (2 * q < NGd) x0 = xb[2 * q];
            if (2 * q + 1 < NGd) x1 = xb[2 * q + 1];
        }
        float wv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = tt0 + i;
            float v = 0.0f;
            if (t < T) {
                if (sh)
                    v = a.has_sgate ? 1.0f / (1.0f + expf(-a.sg_logit[t])) : 1.0f;
                else
                    v = a.route->wt[u][t];
            }
            wv[i] = v;
        }
        // weights, scales, biases of rows h
        const __amdgpu_buffer_rsrc_t rw = vmi_rsrc(md.w + (size_t)slot * H * I8, (uint32_t)H * (I / 2));
        const __amdgpu_buffer_rsrc_t rs = vmi_rsrc(md.s + (size_t)slot * H * NGd, (uint32_t)H * NGd * 2u);
        const __amdgpu_buffer_rsrc_t rb = vmi_rsrc(md.b + (size_t)slot * H * NGd, (uint32_t)H * NGd * 2u);
        vmi_u4 W[NMD];
#pragma unroll
        for (int m = 0; m < NMD; ++m) {
            const uint32_t off = 64u * m + 16u * q;
            W[m] = vmi_bload_b128(rw, off < (uint32_t)(I / 2) ? (uint32_t)h * (I / 2) + off : VMI_OOB, 0);
        }
        uint32_t s0[NMD], s1[NMD];
#pragma unroll
        for (int m = 0; m < NMD; ++m) {
            const int g0 = 2 * m + par;
            s0[m] = vmi_bload_b16(rs, g0 < NGd ? (uint32_t)(h * NGd + g0) * 2u : VMI_OOB, 0);
            if constexpr (!PACK) {
                const int g1 = 2 * m + 1;
                s1[m] = vmi_bload_b16(rs, g1 < NGd ? (uint32_t)(h * NGd + g1) * 2u : VMI_OOB, 0);
            }
        }
        const uint32_t b0 = vmi_bload_b16(rb, 2 * q < NGd ? (uint32_t)(h * NGd + 2 * q) * 2u : VMI_OOB, 0);
        const uint32_t b1 = vmi_bload_b16(rb, 2 * q + 1 < NGd ? (uint32_t)(h * NGd + 2 * q + 1) * 2u : VMI_OOB, 0);

        float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int m = 0; m < NMD; ++m) {
            if constexpr (PACK) {
                vmi_f4 d = zf;
#pragma unroll
                for (int j = 0; j < 4; ++j) d = vmi_mfma_f16(A[m][j], vmi_unpack_u4_f16(W[m][j]), d);
                const float sc = vmi_bf16_to_f32(s0[m]) * kTwo24;
                const float fi[4] = {ifa0[m].x, ifa0[m].y, ifa0[m].z, ifa0[m].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) y[i] = fmaf((tt0 + i < T) ? sc * fi[i] : 0.0f, d[i], y[i]);
            } else {
                vmi_f4 d0 = zf, d1 = zf;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const vmi_u4 bw = vmi_unpack_u4_f16(W[m][j]);
                    d0 = vmi_mfma_f16(q < 2 ? A[m][j] : zero4, bw, d0);
                    d1 = vmi_mfma_f16(q < 2 ? zero4 : A[m][j], bw, d1);
                }
                const float sc0 = vmi_bf16_to_f32(s0[m]) * kTwo24, sc1 = vmi_bf16_to_f32(s1[m]) * kTwo24;
                const float f0[4] = {ifa0[m].x, ifa0[m].y, ifa0[m].z, ifa0[m].w};
                const float f1[4] = {ifa1[m].x, ifa1[m].y, ifa1[m].z, ifa1[m].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool ok = tt0 + i < T;
                    y[i] = fmaf(ok ? sc0 * f0[i] : 0.0f, d0[i], y[i]);
                    y[i] = fmaf(ok ? sc1 * f1[i] : 0.0f, d1[i], y[i]);
                }
            }
        }
        const vmi_f4 db = vmi_mfma_bf16(bias_a_operand(x0, x1), bias_b_operand(b0 | (b1 << 16)), zf);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v = y[i];
            if constexpr (PACK) v += __shfl_xor(v, 32, VMI_WAVE);
            wsum[i] = fmaf(wv[i], v + db[i], wsum[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) s_red[w][i][lane] = wsum[i];
    __syncthreads();
    if (tid < 16 * T) {
        const int t = tid >> 4, rr = tid & 15;
        const int l = 16 * (t >> 2) + rr, i = t & 3;
        float acc = 0.0f;
#pragma unroll
        for (int ww = 0; ww < kDownWaves; ++ww) acc += s_red[ww][i][l];
        const size_t o = (size_t)t * H + blockIdx.x * 16 + rr;
        if (a.residual) acc += vmi_bf16_to_f32(a.residual[o]);
        if (a.out_dtype == VMI_BF16)
            reinterpret_cast<uint16_t*>(a.out)[o] = vmi_f32_to_bf16(acc);
        else
            reinterpret_cast<float*>(a.out)[o] = acc;
    }
}

// --------------------------------------------------------------- prep (slots API)
struct PrepArgs {
    const void* x;
    int T, H;
    OperandOut ops;
};

template <typename XT, int CPL>
__global__ __launch_bounds__(kThreads) void k_prep(PrepArgs a) {
    const int t = blockIdx.x;
    write_operands<XT, CPL>(reinterpret_cast<const XT*>(a.x) + (size_t)t * a.H, nullptr, 0.0f, a.H, t, a.ops);
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

template <bool PACK>
hipError_t launch_gateup_t(const GateUpArgs& ga, int H, hipStream_t s) {
    const int NC = ga.I / kSlice;
    const dim3 grid((ga.has_shared ? NC : 0) + ga.npairs * NC);
    switch (H) {
        case 512: hipLaunchKernelGGL((k_gateup<4, PACK>), grid, dim3(kThreads), 0, s, ga); break;
        case 1024: hipLaunchKernelGGL((k_gateup<8, PACK>), grid, dim3(kThreads), 0, s, ga); break;
        default: hipLaunchKernelGGL((k_gateup<16, PACK>), grid, dim3(kThreads), 0, s, ga); break;
    }
    return hipGetLastError();
}

hipError_t launch_gateup(const GateUpArgs& ga, int H, hipStream_t s) {
    return ga.T <= 8 ? launch_gateup_t<true>(ga, H, s) : launch_gateup_t<false>(ga, H, s);
}

template <bool PACK>
hipError_t launch_downcomb_t(const DownArgs& da, hipStream_t s) {
    const dim3 grid(da.H / 16);
    switch ((da.I + 127) / 128) {
        case 1: hipLaunchKernelGGL((k_downcomb<1, PACK>), grid, dim3(kDownThreads), 0, s, da); break;
        case 2: hipLaunchKernelGGL((k_downcomb<2, PACK>), grid, dim3(kDownThreads), 0, s, da); break;
        case 3: hipLaunchKernelGGL((k_downcomb<3, PACK>), grid, dim3(kDownThreads), 0, s, da); break;
        default: hipLaunchKernelGGL((k_downcomb<4, PACK>), grid, dim3(kDownThreads), 0, s, da); break;
    }
    return hipGetLastError();
}

hipError_t launch_downcomb(const DownArgs& da, hipStream_t s) {
    return da.T <= 8 ? launch_downcomb_t<true>(da, s) : launch_downcomb_t<false>(da, s);
}

template <typename XT>
void launch_prep(const PrepArgs& pa, hipStream_t s) {
    const dim3 grid(pa.T);
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
    const size_t nact = (size_t)T * k + 1;  // distinct slots + the shared expert
    w.status = reinterpret_cast<uint32_t*>(take(256));
    w.route = reinterpret_cast<RouteInfo*>(take(sizeof(RouteInfo)));
    w.logits = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T * (num_experts > 0 ? num_experts : 1)));
    w.sg_logit = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.xop = reinterpret_cast<vmi_u4*>(take(sizeof(uint16_t) * (size_t)T * hidden));
    w.xsum = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T * (hidden / 64)));
    w.fscale = reinterpret_cast<float*>(take(sizeof(float) * (size_t)T));
    w.actop = reinterpret_cast<vmi_u4*>(take(sizeof(uint16_t) * nact * T * inter));
    w.axs = reinterpret_cast<float*>(take(sizeof(float) * nact * T * (inter / 64)));
    w.aifa = reinterpret_cast<float*>(take(sizeof(float) * nact * (inter / 64) * kTPad));
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
        return vmi::fail(VMI_ERR_INVALID, "weight arrays must be non-null and 16-byte aligned");
    if (cap <= 0) return vmi::fail(VMI_ERR_INVALID, "cap=%d", cap);
    const vmi::MoeWorkspace ws = vmi::carve_workspace(workspace, T, k, hidden, inter, 0);
    if (!workspace || workspace_bytes < ws.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", ws.bytes, workspace_bytes);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const OperandOut ops{ws.xop, ws.xsum, ws.fscale};

    const PrepArgs pa{x, T, hidden, ops};
    if (x_dtype == VMI_BF16)
        launch_prep<uint16_t>(pa, s);
    else
        launch_prep<float>(pa, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_prep launch");

    GateUpArgs ga{};
    ga.T = T; ga.I = inter; ga.k = k; ga.E = 0; ga.npairs = T * k; ga.has_shared = 0;
    ga.from_slots = 1; ga.norm = 1; ga.cap = cap;
    ga.slots = local_slots; ga.in_scores = scores;
    ga.gate = gate; ga.up = up; ga.sh_gate = gate; ga.sh_up = up;
    ga.xop = ws.xop; ga.xsum = ws.xsum; ga.fscale = ws.fscale;
    ga.route = ws.route; ga.status = ws.status;
    ga.actop = ws.actop; ga.axs = ws.axs; ga.aifa = ws.aifa;
    e = launch_gateup(ga, hidden, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_gateup launch");

    DownArgs da{};
    da.T = T; da.H = hidden; da.I = inter; da.npairs = T * k; da.has_shared = 0; da.has_sgate = 0;
    da.route = ws.route; da.down = down; da.sh_down = down;
    da.actop = ws.actop; da.axs = ws.axs; da.aifa = ws.aifa;
    da.residual = nullptr; da.out = out; da.out_dtype = out_dtype;
    e = launch_downcomb(da, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_downcomb launch");
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
        return vmi::fail(VMI_ERR_INVALID, "router/gate/up/down arrays must be non-null and 16-byte aligned");
    if (has_shared && (!qmat_ok(D.shared_gate) || !qmat_ok(D.shared_up) || !qmat_ok(D.shared_down)))
        return vmi::fail(VMI_ERR_INVALID, "shared expert arrays must be non-null and 16-byte aligned");
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
    constexpr int rows_per_wg = kRouterRowsPerWave * (kThreads / VMI_WAVE);
    ra.row_wgs = (D.num_experts + has_sgate + rows_per_wg - 1) / rows_per_wg;
    ra.logits = ws.logits; ra.sg_logit = ws.sg_logit; ra.ops = ops;
    const dim3 rgrid(ra.row_wgs + T);
    switch (D.hidden) {
        case 512: hipLaunchKernelGGL(k_router<8>, rgrid, dim3(kThreads), 0, s, ra); break;
        case 1024: hipLaunchKernelGGL(k_router<16>, rgrid, dim3(kThreads), 0, s, ra); break;
        default: hipLaunchKernelGGL(k_router<32>, rgrid, dim3(kThreads), 0, s, ra); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_router launch");

    GateUpArgs ga{};
    ga.T = T; ga.I = D.inter; ga.k = D.top_k; ga.E = D.num_experts; ga.npairs = T * D.top_k;
    ga.has_shared = has_shared; ga.from_slots = 0; ga.norm = D.norm_topk_prob; ga.cap = D.cap;
    ga.logits = ws.logits; ga.table = D.slot_table;
    ga.gate = D.gate; ga.up = D.up;
    ga.sh_gate = has_shared ? D.shared_gate : D.gate;
    ga.sh_up = has_shared ? D.shared_up : D.up;
    ga.xop = ws.xop; ga.xsum = ws.xsum; ga.fscale = ws.fscale;
    ga.route = ws.route; ga.status = ws.status; ga.ids_out = ids_out; ga.scores_out = scores_out;
    ga.actop = ws.actop; ga.axs = ws.axs; ga.aifa = ws.aifa;
    e = launch_gateup(ga, D.hidden, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_gateup launch");

    DownArgs da{};
    da.T = T; da.H = D.hidden; da.I = D.inter; da.npairs = T * D.top_k;
    da.has_shared = has_shared; da.has_sgate = has_sgate;
    da.route = ws.route; da.down = D.down; da.sh_down = has_shared ? D.shared_down : D.down;
    da.actop = ws.actop; da.axs = ws.axs; da.aifa = ws.aifa; da.sg_logit = ws.sg_logit;
    da.residual = residual; da.out = out; da.out_dtype = VMI_BF16;
    e = launch_downcomb(da, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "k_downcomb launch");
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
