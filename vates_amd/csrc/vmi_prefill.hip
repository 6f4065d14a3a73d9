// Expert-major prefill of one MoE layer (long prompts, T up to 65536 tokens).
//
// The reference computes a long prefill by expert groups
// (mlx_streaming/core/moe/block.py:111-243): histogram of routed experts,
// argsort, per-expert gathers of the routed token rows, SwitchGLU on each
// group, and a deterministic scatter of the weighted results in route-rank
// order (core/moe/custom_kernel.py:20-118).  With every expert resident in HBM
// there is no group-size bound to respect, so one pass covers the layer:
//
//   k_pf_prep     per token: optional RMSNorm, MFMA operands of x (fp16, range
//                 factor per token), per-group operand sums for the router's
//                 affine term, the shared-expert gate logit; clears counters
//   k_pf_router3  router logits [T, E] as a tiled MFMA GEMM on the 4/8-bit
//                 router (weights enter the MFMA as exact fp16 subnormals),
//                 in two halves of K that the top-k adds
//   k_pf_topk     one wave per token: top-k, softmax, renorm, slot table
//   k_pf_count    routes per slot and each route's rank in its slot
//   k_pf_place    exclusive scans of the counts (each workgroup), every
//                 routed (token, rank) into its slot's list, the list of
//                 128-route tiles
//   k_pf_table    per touched expert (and the shared one): the fp16
//                 dequantisation table of its gate, up and down rows
//   k_pf_gateup3  per (M tile, 256 intermediate rows): gate and up MFMA GEMMs
//                 over the tile's gathered tokens, SwiGLU rounded to bf16,
//                 the activations as fp16 operands times 2^-E (E per route
//                 and 256-column block)
//   k_pf_down3    per (M tile, 512 hidden rows): down MFMA GEMM, times the
//                 route's combine weight, one bf16 row per (token, rank)
//   k_pf_combine  out[t] = sum over ranks 0..k (rank k: the gated shared
//                 expert) in rank order, fp32, + residual
//
// Route (token t, rank j) owns row t*(k+1) + j of the activation and result
// buffers, so no result depends on the order in which assignments are placed:
// the layer is bit-deterministic run to run.
//
// 4-bit weights unpack as exact fp16 subnormals q 2^-24 (nibble masks, slot
// order {0,4,1,5,2,6,3,7}, the odd nibbles carrying 16 q and the other operand
// divided by 16 there).  The expert GEMMs dequantise them in fp16 with the
// group's scale and bias folded in (one packed FMA per two values), so their
// MFMAs accumulate the whole affine product over K; the router keeps the
// exact operand, applies each group's scale to the group's MFMA result (FMA)
// and adds the bias through per-group operand sums, so its logits stay exact
// enough for the top-k.

#include <type_traits>

#include "vmi_device.h"
#include "vmi_internal.h"

VMI_TL_DECL

namespace {

constexpr int kPfThreads = 256;
constexpr int kTM3 = 128;    // routes per tile of the expert GEMMs
constexpr int kPfMaxE = 1024;
constexpr int kPfMaxK = 16;

__device__ __forceinline__ int pf_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

struct PfArgs {
    int T, H, I, E, k, cap, norm_topk, router_bits, sg_bits, has_shared, has_sgate;
    const uint16_t* x;          // [T, H] bf16
    const uint16_t* norm_w;     // [H] or null
    float eps;
    const uint16_t* residual;   // [T, H] or null
    vmi_qmat router;            // [E, H]
    const float* logit_bias;    // [E] or null
    const int32_t* table;       // [E] or null
    vmi_qmat gate, up, down;    // [cap, ...]: gate/up words MFMA-major, down group-major [cap, I/64, H, 8 words]
    vmi_qmat sh_gate, sh_up, sh_down, sgate;
    // workspace
    vmi_u4* xop4;               // [T, H/8] fp16 operands, 4-bit slot order
    float* xsum4;               // [T, H/64] per group, the sum of what the router MFMAs multiply
    float* fscale;              // [T]
    float* logits;              // [2, T, E]: the router's two halves of K
    float* sglogit;             // [T]
    int32_t* ids;               // [T, k]
    float* scores;              // [T, k]
    int32_t* slots;             // [T, k] (-1: invalid)
    int32_t* counts;            // [cap]
    int32_t* fill;              // [T*k] rank of each route inside its slot
    int4* tiles;                // [max_tiles]: slot (-1 shared), list start (or token start), rows, 0
    int32_t* ntiles;            // [1]
    int32_t* list;              // [T*k] route rows t*(k+1)+j grouped by slot
    uint32_t* tgu;              // [cap+1, H/128, 2, I, 2] fp16 (s', b') of gate/up rows per group pair (slot cap: shared)
    float* pgu;                 // [cap+1, 2, I] 2^(24-P) per gate/up row
    uint32_t* tdn;              // [cap+1, ceil(I/128), H, 2] the same for down rows
    float* pdn;                 // [cap+1, H]
    vmi_u4* actop;              // [T*(k+1), I/8] fp16 operands (times 2^-E), 4-bit slot order
    int32_t* aexp;              // [T*(k+1), ceil(I/256)]: E of each route and 256-column block
    uint16_t* ybuf;             // [T*(k+1), H] bf16 weighted expert outputs
    uint16_t* out;              // [T, H]
    uint32_t* status;
    int32_t* ids_out;
    float* scores_out;
    int max_tiles;
};

// ------------------------------------------------------------------ prep
// fp16 operand of 8 columns for 4-bit words: slots {0,4,1,5,2,6,3,7}, odd
// nibble slots divided by 16; with SUM, s accumulates what the MFMA
// multiplies (the 4-bit router's affine term needs it).
template <bool SUM>
__device__ __forceinline__ vmi_u4 op4(const float (&v)[8], float f, float& s) {
    const _Float16 h0 = (_Float16)(v[0] * f), h1 = (_Float16)(v[4] * f);
    const _Float16 h2 = (_Float16)(v[1] * f * 0.0625f), h3 = (_Float16)(v[5] * f * 0.0625f);
    const _Float16 h4 = (_Float16)(v[2] * f), h5 = (_Float16)(v[6] * f);
    const _Float16 h6 = (_Float16)(v[3] * f * 0.0625f), h7 = (_Float16)(v[7] * f * 0.0625f);
    if constexpr (SUM)
        s += (float)h0 + (float)h1 + (float)h4 + (float)h5 + 16.0f * ((float)h2 + (float)h3 + (float)h6 + (float)h7);
    vmi_u4 r;
    r[0] = vmi_h2_bits(h0, h1);
    r[1] = vmi_h2_bits(h2, h3);
    r[2] = vmi_h2_bits(h4, h5);
    r[3] = vmi_h2_bits(h6, h7);
    return r;
}

typedef _Float16 pf_h2v __attribute__((ext_vector_type(2)));

// Eight 8-bit values of two packed words (columns 0..3, 4..7) as exact fp16
// subnormals n * 2^-24 in the operand's slot order {0,4,1,5,2,6,3,7}, the
// odd slots times 16 (exact) to match the operand's odd slots divided by 16.
__device__ __forceinline__ vmi_u4 unpack_u8_f16(uint32_t w0, uint32_t w1) {
    vmi_u4 r;
    r[0] = __builtin_amdgcn_perm(w1, w0, 0x0C040C00u);
    r[1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(pf_h2v, __builtin_amdgcn_perm(w1, w0, 0x0C050C01u)) *
                                            (pf_h2v){16.0f16, 16.0f16});
    r[2] = __builtin_amdgcn_perm(w1, w0, 0x0C060C02u);
    r[3] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(pf_h2v, __builtin_amdgcn_perm(w1, w0, 0x0C070C03u)) *
                                            (pf_h2v){16.0f16, 16.0f16});
    return r;
}

__device__ __forceinline__ void bf16x8(const uint4& q, float (&v)[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

// Shared-expert gate logit of one token by its wave (lane l: the same
// columns as its operand words u), on the effective fp16 operands (x * f) and
// the dequantised gate row, in a fixed order, canonical wave sum; the caller
// divides by f.
template <int NCH>
__device__ __forceinline__ float pf_sgate_dot(const vmi_u4 (&u)[NCH], const PfArgs& a) {
    const int lane = threadIdx.x & 63;
    const int bits = a.sg_bits;
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
        // op4 slot s holds column {0,4,1,5,2,6,3,7}[s]; odd columns carry /16
        float xv[8];
        const _Float16 h[8] = {
            __builtin_bit_cast(_Float16, (uint16_t)(u[c][0] & 0xffffu)), __builtin_bit_cast(_Float16, (uint16_t)(u[c][0] >> 16)),
            __builtin_bit_cast(_Float16, (uint16_t)(u[c][1] & 0xffffu)), __builtin_bit_cast(_Float16, (uint16_t)(u[c][1] >> 16)),
            __builtin_bit_cast(_Float16, (uint16_t)(u[c][2] & 0xffffu)), __builtin_bit_cast(_Float16, (uint16_t)(u[c][2] >> 16)),
            __builtin_bit_cast(_Float16, (uint16_t)(u[c][3] & 0xffffu)), __builtin_bit_cast(_Float16, (uint16_t)(u[c][3] >> 16))};
        xv[0] = (float)h[0];
        xv[4] = (float)h[1];
        xv[1] = 16.0f * (float)h[2];
        xv[5] = 16.0f * (float)h[3];
        xv[2] = (float)h[4];
        xv[6] = (float)h[5];
        xv[3] = 16.0f * (float)h[6];
        xv[7] = 16.0f * (float)h[7];
        const int c0 = 8 * (lane * NCH + c);  // first column of this word
        const int gi = c0 >> 6;
        const float sc = vmi_bf16_to_f32(a.sgate.s[gi]), bi = vmi_bf16_to_f32(a.sgate.b[gi]);
        uint32_t qv[8];
        if (bits == 4) {
            const uint32_t wd = a.sgate.w[c0 >> 3];
#pragma unroll
            for (int i = 0; i < 8; ++i) qv[i] = (wd >> (4 * i)) & 0xFu;
        } else {
            const uint32_t w0 = a.sgate.w[c0 >> 2], w1 = a.sgate.w[(c0 >> 2) + 1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qv[i] = (w0 >> (8 * i)) & 0xFFu;
                qv[4 + i] = (w1 >> (8 * i)) & 0xFFu;
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) acc = fmaf(xv[i], fmaf((float)qv[i], sc, bi), acc);
    }
    return vmi_wave_sum_canon(acc);
}

// One wave per token; lane l owns columns [l*H/64, (l+1)*H/64) (H/512 chunks
// of 8).  RMSNorm (canonical order) when norm_w, range factor, operands, and
// the shared-expert gate logit from those operands.
template <int NCH>
__global__ __launch_bounds__(kPfThreads) void k_pf_prep(PfArgs a) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (kPfThreads / 64) + pf_wave();
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < a.cap; i += kPfThreads) a.counts[i] = 0;
    if (t >= a.T) return;
    constexpr int cpl = 8 * NCH;
    const uint16_t* xr = a.x + (size_t)t * a.H + lane * cpl;
    float v[NCH][8];
#pragma unroll
    for (int c = 0; c < NCH; ++c) bf16x8(*reinterpret_cast<const uint4*>(xr + 8 * c), v[c]);
    if (a.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int c = 0; c < NCH; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = fmaf(v[c][i], v[c][i], ss);
        ss = vmi_wave_sum_canon(ss);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / (float)a.H) + a.eps));
        const uint16_t* nw = a.norm_w + lane * cpl;
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            float g[8];
            bf16x8(*reinterpret_cast<const uint4*>(nw + 8 * c), g);
            // rounded to bf16 in pairs (v_cvt_pk_bf16_f32: the bits of
            // vmi_f32_to_bf16 for every non-NaN value)
#pragma unroll
            for (int i = 0; i < 8; i += 2) {
                const uint32_t pk = vmi_pack_bf16x2((v[c][i] * inv) * g[i], (v[c][i + 1] * inv) * g[i + 1]);
                v[c][i] = __uint_as_float(pk << 16);
                v[c][i + 1] = __uint_as_float(pk & 0xffff0000u);
            }
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c)
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
    amax = vmi_wave_max(amax);
    const float f = vmi_fp16_range_scale(amax);
    // group of 64 columns = 8 chunks: lanes (8 / NCH) per group
    constexpr int LPG = 8 / NCH;
    float s4 = 0.0f;
    const size_t orow = (size_t)t * (a.H / 8) + lane * NCH;
    vmi_u4 u[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) u[c] = op4<true>(v[c], f, s4);
#pragma unroll
    for (int c = 0; c < NCH; ++c) a.xop4[orow + c] = u[c];
    // lanes of one group sum their partials in lane order
#pragma unroll
    for (int o = 1; o < LPG; o <<= 1) s4 += __shfl_xor(s4, o);
    if ((lane % LPG) == 0) a.xsum4[(size_t)t * (a.H / 64) + lane / LPG] = s4;
    if (lane == 0) a.fscale[t] = f;
    if (a.has_sgate) {
        const float sg = pf_sgate_dot<NCH>(u, a);
        if (lane == 0) a.sglogit[t] = sg / f;
    }
}

// ------------------------------------------------------- grouped GEMM core
// One wave accumulates 16 (rows) x 16 (output features) tiles over the
// quantisation groups of K: per group two MFMAs with the group's weights as
// exact subnormals, then acc += D * scale * 2^24 (+ the affine-bias term).
// Lane l: A row m = l%16 (rows of the tile), K block q = l/16; B column
// n = l%16; D rows 4q + r, column n.

// ------------------------------------------------------------------ top-k
__device__ __forceinline__ uint64_t pf_rank_key(float f, int e) {
    uint32_t u = __float_as_uint(f);
    u = (u == 0x80000000u) ? 0u : u;
    const uint32_t ok = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    const uint32_t hi = (f != f) ? 1u : ok;
    return ((uint64_t)hi << 32) | (uint32_t)(0xffffffffu - (uint32_t)e);
}

// One wave per token (block.py:321-329): lane l holds experts l + 64 i
// (i < E/64 <= 16) as rank keys, sorted descending once (bitonic network);
// each of the k rounds takes the wave-wide maximum of the lanes' head values
// (the full (value, index) key only when values tie) and the winning lane
// records the expert and pops its head.
template <int NI>
__global__ __launch_bounds__(kPfThreads) void k_pf_topk(PfArgs a) {
    __shared__ int s_sel[kPfThreads / 64][kPfMaxK];  // a wave's winners in round order
    const int lane = threadIdx.x & 63, w = pf_wave();
    const int t = blockIdx.x * (kPfThreads / 64) + w;
    if (t >= a.T) return;  // whole waves; nothing below synchronises the workgroup
    // the logit is the sum of the router's two halves of K, in that order
    const float* lt = a.logits + (size_t)t * a.E;
    const float* lt2 = lt + (size_t)a.T * a.E;
    const int nreal = a.E >> 6;  // key slots i < E/64 are real (uniform)
    float lv[NI];
    uint64_t key[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        lv[i] = i < nreal ? lt[lane + 64 * i] + lt2[lane + 64 * i] : 0.0f;
        key[i] = i < nreal ? pf_rank_key(lv[i], lane + 64 * i) : 0ull;
    }
#pragma unroll
    for (int size = 2; size <= NI; size *= 2)
#pragma unroll
        for (int stride = size / 2; stride > 0; stride /= 2)
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const int j = i ^ stride;
                if (j > i) vmi_cx64(key[i], key[j], (i & size) == 0);
            }
#pragma unroll 1
    for (int j = 0; j < a.k; ++j) {
        const uint32_t hv = (uint32_t)(key[0] >> 32);
        const uint32_t Mv = vmi_wave_max_u32(hv);
        const uint64_t cand = __ballot(hv == Mv);
        bool win;
        if (__popcll(cand) == 1) {
            win = hv == Mv;
        } else {
            const uint64_t M = vmi_wave_max_u64(hv == Mv ? key[0] : 0ull);
            win = key[0] == M;
        }
        if (win) {
            s_sel[w][j] = (int)(0xffffffffu - (uint32_t)key[0]);
#pragma unroll
            for (int i = 0; i + 1 < NI; ++i) key[i] = key[i + 1];
            key[NI - 1] = 0ull;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool sel = lane < a.k;
    const int my_idx = sel ? s_sel[w][lane] : 0;
    const float my_val = sel ? lt[my_idx] + lt2[my_idx] : 0.0f;
    const float mx = vmi_readlane_f32(my_val, 0);
    const bool bad = __ballot(sel && !(fabsf(my_val) < 3.0e38f)) != 0;
    const float e = sel ? expf(my_val - mx) : 0.0f;
    float den = 0.0f;
    if (a.norm_topk) {
        for (int j = 0; j < a.k; ++j) den = den + vmi_readlane_f32(e, j);
    } else {
        float part = 0.0f;
#pragma unroll
        for (int i = 0; i < NI; ++i)
            if (i < nreal) part = part + expf(lv[i] - mx);
        den = vmi_wave_sum_canon(part);
    }
    if (sel) {
        const float sc = e / den;
        const int slot = a.table ? a.table[my_idx] : my_idx;
        const bool ok = slot >= 0 && slot < a.cap;
        a.ids[t * a.k + lane] = my_idx;
        a.scores[t * a.k + lane] = sc;
        a.slots[t * a.k + lane] = ok ? slot : -1;
        if (a.ids_out) a.ids_out[t * a.k + lane] = my_idx;
        if (a.scores_out) a.scores_out[t * a.k + lane] = sc;
        if (!ok) atomicOr(a.status, VMI_STATUS_BAD_SLOT);
    }
    if (bad && lane == 0) atomicOr(a.status, VMI_STATUS_BAD_ROUTE);
}

// ------------------------------------------------------------ scan, place
// Exclusive prefix sums over the slots (cap <= 1024) of the route counts and
// of their 128-route tile counts, by one workgroup of kPfThreads threads into
// LDS: thread i takes slots 4i..4i+3, the waves scan their lanes' sums, then
// the wave totals.  Returns the routed tiles in all.
__device__ int pf_slot_scan(const PfArgs& a, int* s_off, int* s_toff) {
    __shared__ int s_wsum[kPfThreads / 64][2];
    const int tid = threadIdx.x, lane = tid & 63, w = pf_wave();
    int c[4], cs = 0, ts = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int slot = 4 * tid + i;
        c[i] = slot < a.cap ? a.counts[slot] : 0;
        cs += c[i];
        ts += (c[i] + kTM3 - 1) / kTM3;
    }
    // inclusive wave scans of the thread sums
    int ic = cs, it = ts;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int vc = __shfl_up(ic, o), vt = __shfl_up(it, o);
        if (lane >= o) {
            ic += vc;
            it += vt;
        }
    }
    if (lane == 63) {
        s_wsum[w][0] = ic;
        s_wsum[w][1] = it;
    }
    __syncthreads();
    int bc = 0, bt = 0, total_t = 0;
#pragma unroll
    for (int v = 0; v < kPfThreads / 64; ++v) {
        if (v < w) {
            bc += s_wsum[v][0];
            bt += s_wsum[v][1];
        }
        total_t += s_wsum[v][1];
    }
    int oc = bc + ic - cs, ot = bt + it - ts;  // exclusive
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s_off[4 * tid + i] = oc;
        s_toff[4 * tid + i] = ot;
        oc += c[i];
        ot += (c[i] + kTM3 - 1) / kTM3;
    }
    __syncthreads();
    return total_t;
}

// Routes per slot and each route's rank inside its slot: a block counts its
// kCountRoutes routes in LDS, then adds one total per slot it touched to the
// global count, whose old value is the block's base.  (Popular slots see one
// global atomic per block instead of one per route.)  The rank order inside a
// slot is arrival order; no result depends on it.
constexpr int kCountRoutes = 2048;
__global__ __launch_bounds__(kPfThreads) void k_pf_count(PfArgs a) {
    __shared__ int s_cnt[1024];
    __shared__ int s_base[1024];
    const int tid = threadIdx.x;
    for (int i = tid; i < a.cap; i += kPfThreads) s_cnt[i] = 0;
    __syncthreads();
    const int p0 = blockIdx.x * kCountRoutes, n = min(kCountRoutes, a.T * a.k - p0);
    int local[kCountRoutes / kPfThreads];
#pragma unroll
    for (int i = 0; i < kCountRoutes / kPfThreads; ++i) {
        const int p = tid + i * kPfThreads;
        local[i] = -1;
        if (p < n) {
            const int slot = a.slots[p0 + p];
            if (slot >= 0) local[i] = atomicAdd(&s_cnt[slot], 1);
        }
    }
    __syncthreads();
    for (int i = tid; i < a.cap; i += kPfThreads)
        s_base[i] = s_cnt[i] ? atomicAdd(&a.counts[i], s_cnt[i]) : 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kCountRoutes / kPfThreads; ++i) {
        const int p = tid + i * kPfThreads;
        if (p < n && local[i] >= 0) a.fill[p0 + p] = s_base[a.slots[p0 + p]] + local[i];
    }
}

// Every valid route into its slot's list at offset[slot] + rank, every
// workgroup scanning the slot counts itself (no separate scan launch);
// workgroup 0 also writes the list of 128-route tiles (the shared expert's
// last).
__global__ __launch_bounds__(kPfThreads) void k_pf_place(PfArgs a) {
    static_assert(4 * kPfThreads >= 1024, "four slots per thread cover cap <= 1024");
    __shared__ int s_off[4 * kPfThreads];
    __shared__ int s_toff[4 * kPfThreads];
    const int routed_tiles = pf_slot_scan(a, s_off, s_toff);
    const int tid = threadIdx.x;
    if (blockIdx.x == 0) {
        for (int slot = tid; slot < a.cap; slot += kPfThreads) {
            const int c = a.counts[slot], off = s_off[slot], toff = s_toff[slot];
            for (int i = 0; i * kTM3 < c; ++i)
                a.tiles[toff + i] = make_int4(slot, off + i * kTM3, min(kTM3, c - i * kTM3), 0);
        }
        const int sh_tiles = a.has_shared ? (a.T + kTM3 - 1) / kTM3 : 0;
        for (int i = tid; i < sh_tiles; i += kPfThreads)
            a.tiles[routed_tiles + i] = make_int4(-1, i * kTM3, min(kTM3, a.T - i * kTM3), 0);
        if (tid == 0) a.ntiles[0] = routed_tiles + sh_tiles;
    }
    const int p = blockIdx.x * kPfThreads + tid;
    if (p >= a.T * a.k) return;
    const int slot = a.slots[p];
    if (slot < 0) return;
    const int t = p / a.k, j = p - t * a.k;
    a.list[s_off[slot] + a.fill[p]] = t * (a.k + 1) + j;
}

// Route row of tile row i (or -1 past the tile).
__device__ __forceinline__ int tile_route(const PfArgs& a, const int4& tl, int i) {
    if (i >= tl.z) return -1;
    return tl.x >= 0 ? a.list[tl.y + i] : (tl.y + i) * (a.k + 1) + a.k;
}

constexpr int kMaxG = 32;  // quantisation groups along K (K <= 2048)

// s_waitcnt vmcnt(N): the GEMMs' LDS copies are inline assembly the
// compiler does not count, so the ring orders them itself.

template <int N>
__device__ __forceinline__ void pf_wait_vmcnt() {
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Byte offset of 8-byte unit `unit8` (0..3) of packed weight row `row` inside
// a slot: the row's 16-byte halves are swapped when bit 3 of the row is set,
// so the 8-byte operand reads of 16 consecutive rows hit distinct banks.
__device__ __forceinline__ uint32_t ring_off(int row, int unit8) {
    return 32u * row + 16u * (((unsigned)unit8 >> 1) ^ (((unsigned)row >> 3) & 1u)) + 8u * (unit8 & 1);
}

// ----------------------------------------------- tiled MFMA GEMMs
// The tile GEMMs stream K one quantisation group (64 values) per stage
// through LDS slots filled by global_load_lds, each thread moving whole
// 16-byte pieces: the A operands (128 rows x 128 bytes, fp16) and the packed
// weight rows (32 bytes each).  An A row r keeps its 16-byte piece c at
// position c ^ ((r >> 1) & 7) (pf_a_off), so the 16 rows of one ds_read_b128
// phase cover the 64 banks once; a weight row keeps the half-swap on bit 3 of
// the row (ring_off).  The router (k_pf_router3) runs four waves in a 2 x 2
// grid over a ring of kPfStages slots; the expert GEMMs (k_pf_gateup3,
// k_pf_down3) run eight waves side by side with their own slot layout.
// Workgroup L runs tile 8*(L/8/NB) + L%8 and column block (L/8)%NB: the
// column blocks of one tile share an XCD, so its A rows reach that L2 once.
constexpr int kPfStages = 2;   // LDS ring depth: kPfStages - 1 groups in flight
constexpr int kPfA = kTM3 * 128;

__device__ __forceinline__ void pf_tile_of(int L, int nb_count, int& ti, int& nb) {
    const int xcd = L & 7, idx = L >> 3;
    ti = 8 * (idx / nb_count) + xcd;
    nb = idx % nb_count;
}

// byte offset of A row r, logical 16-byte piece c, inside a slot.  Rows are
// 128 bytes (half of the 64 four-byte banks), so rows r and r + 1 take the
// two bank halves and the piece is swizzled by bits 1..3 of the row: the 16
// rows a ds_read_b128 of one piece touches (16 lanes) then cover all 64 banks
// once.
__device__ __forceinline__ uint32_t pf_a_off(int r, int c) {
    return 16u * (8u * r + (unsigned)(c ^ ((r >> 1) & 7)));
}
// the logical piece a slot position holds (the inverse of pf_a_off's swizzle)
__device__ __forceinline__ int pf_a_piece(int r, int pos) { return pos ^ ((r >> 1) & 7); }

// The eight 4-bit values of one packed word, dequantised in fp16 by one
// packed FMA per two values: (q 2^-24) s' + b' with s2 = (s', s'),
// b2 = (b', b') and b16 = 16 b2 (the odd words of vmi_unpack_u4_f16 carry
// 16 q).  The elements are taken into named scalars first: a bit cast of a
// vector element indexed by a loop counter compiled to one element's result
// replicated four times.
__device__ __forceinline__ uint32_t pf_fma_h2(uint32_t x, uint32_t y, uint32_t z) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(pf_h2v, x),
                                                                  __builtin_bit_cast(pf_h2v, y),
                                                                  __builtin_bit_cast(pf_h2v, z)));
}
__device__ __forceinline__ vmi_u4 pf_dequant_f16(uint32_t wq, uint32_t s2, uint32_t b2, uint32_t b16) {
    const vmi_u4 u = vmi_unpack_u4_f16(wq);
    const uint32_t u0 = u.x, u1 = u.y, u2 = u.z, u3 = u.w;
    vmi_u4 r;
    r.x = pf_fma_h2(u0, s2, b2);
    r.y = pf_fma_h2(u1, s2, b16);
    r.z = pf_fma_h2(u2, s2, b2);
    r.w = pf_fma_h2(u3, s2, b16);
    return r;
}

// The weight row's power of two P for the fp16 table: its largest |scale|
// times 2^P below 2^15 (in [2^14, 2^15) unless the biases bind) and its
// largest |bias| times 2^(P-24) below 2^11, so s 2^P and b 2^(P-24) are
// finite and exact in fp16 (bf16 values times powers of two, down to fp16's
// subnormals), 16 b 2^(P-24) (the odd words' bias) is finite too, and a
// dequantised value stays below 2^16.  mxs, mxb: the largest |scale| and
// |bias| as float bits (zero: all zero).  P is kept in [-100, 127], so
// 2^(24-P) is a finite float.
__device__ __forceinline__ int pf_row_pow2(uint32_t mxs, uint32_t mxb) {
    int P = 127, e = 0;
    if (mxs) {
        (void)frexpf(__uint_as_float(mxs), &e);  // mxs = f 2^e, f in [0.5, 1)
        P = min(P, 15 - e);
    }
    if (mxb) {
        (void)frexpf(__uint_as_float(mxb), &e);
        P = min(P, 35 - e);
    }
    return (mxs | mxb) ? max(P, -100) : 0;
}

// (s', b') of a table word -> s2, b2, b16
__device__ __forceinline__ void pf_affine_pairs(uint32_t sbw, uint32_t& s2, uint32_t& b2, uint32_t& b16) {
    s2 = __builtin_amdgcn_perm(sbw, sbw, 0x01000100u);
    b2 = __builtin_amdgcn_perm(sbw, sbw, 0x03020302u);
    b16 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(pf_h2v, b2) * (pf_h2v){16.0f16, 16.0f16});
}

// The fp16 dequantisation tables of every expert the routing touched (and of
// the shared expert, slot cap): per weight row, its power of two P
// (pf_row_pow2) and per group the pair (s 2^P, b 2^(P-24)) as fp16 bits, laid
// out per group pair so a wave's rows of one pair are one contiguous run;
// 2^(24-P) per row.  A thread takes one gate or up row (its scales and biases
// in registers, one pass) or four consecutive down rows (8-byte loads of the
// group-major scales; a second pass reads them again from the cache).
// Column blocks of 512 hidden rows one down workgroup runs in sequence (two
// when the count is even), so the prologue is paid once per pair of blocks.
__host__ __device__ __forceinline__ int pf_down_blocks(int H) { return (H / 512) % 2 == 0 ? 2 : 1; }
__host__ __device__ __forceinline__ int pf_table_blocks(int H, int I) { return (2 * I + H / 4 + kPfThreads - 1) / kPfThreads; }

__global__ __launch_bounds__(kPfThreads) void k_pf_table(PfArgs a) {
    const int I = a.I, H = a.H, G = H / 64, GP = G / 2, Gd = I / 64, GPd = (Gd + 1) / 2;
    const int bps = pf_table_blocks(H, I);
    const int slot = blockIdx.x / bps, r = (blockIdx.x - slot * bps) * kPfThreads + threadIdx.x;
    const bool shared = slot == a.cap;
    if (shared ? !a.has_shared : (a.counts && a.counts[slot] == 0)) return;  // counts null: every slot
    if (r < 2 * I) {
        const int mt = r >= I, row = r - mt * I;
        const vmi_qmat M = mt ? (shared ? a.sh_up : a.up) : (shared ? a.sh_gate : a.gate);
        const uint16_t* sp = M.s + ((shared ? 0 : (size_t)slot) * I + row) * G;
        const uint16_t* bp = M.b + ((shared ? 0 : (size_t)slot) * I + row) * G;
        uint4 sv[kMaxG / 8], bv[kMaxG / 8];
#pragma unroll
        for (int c = 0; c < kMaxG / 8; ++c) {
            sv[c] = c < G / 8 ? *reinterpret_cast<const uint4*>(sp + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
            bv[c] = c < G / 8 ? *reinterpret_cast<const uint4*>(bp + 8 * c) : make_uint4(0u, 0u, 0u, 0u);
        }
        uint32_t mx = 0u, mxb = 0u;  // |scale|, |bias| as float bits: ordered as integers
#pragma unroll
        for (int c = 0; c < kMaxG / 8; ++c) {
            const uint32_t ws[4] = {sv[c].x, sv[c].y, sv[c].z, sv[c].w}, wb[4] = {bv[c].x, bv[c].y, bv[c].z, bv[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                mx = max(mx, max((ws[e] << 16) & 0x7fff0000u, ws[e] & 0x7fff0000u));
                mxb = max(mxb, max((wb[e] << 16) & 0x7fff0000u, wb[e] & 0x7fff0000u));
            }
        }
        const int P = pf_row_pow2(mx, mxb);
        const float ps = ldexpf(1.0f, P), pb = ldexpf(1.0f, P - 24);
        uint32_t* tp = a.tgu + (((size_t)slot * GP * 2 + mt) * I + row) * 2;
#pragma unroll
        for (int c = 0; c < kMaxG / 8; ++c) {
            if (c >= G / 8) break;
            const uint32_t ws[4] = {sv[c].x, sv[c].y, sv[c].z, sv[c].w}, wb[4] = {bv[c].x, bv[c].y, bv[c].z, bv[c].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {  // groups 8c + 2e, 8c + 2e + 1: pair 4c + e
                uint2 o;
                o.x = vmi_h2_bits((_Float16)(vmi_bf16_to_f32(ws[e] & 0xffffu) * ps), (_Float16)(vmi_bf16_to_f32(wb[e] & 0xffffu) * pb));
                o.y = vmi_h2_bits((_Float16)(vmi_bf16_to_f32(ws[e] >> 16) * ps), (_Float16)(vmi_bf16_to_f32(wb[e] >> 16) * pb));
                *reinterpret_cast<uint2*>(tp + (size_t)(4 * c + e) * 4 * I) = o;
            }
        }
        a.pgu[((size_t)slot * 2 + mt) * I + row] = ldexpf(1.0f, 24 - P);
    } else if (r < 2 * I + H / 4) {
        const int h = 4 * (r - 2 * I);  // rows h .. h + 3
        const vmi_qmat Dm = shared ? a.sh_down : a.down;
        const size_t mb = (shared ? 0 : (size_t)slot) * Gd * H + h;
        uint32_t mx[4] = {0u, 0u, 0u, 0u}, mxb[4] = {0u, 0u, 0u, 0u};
        for (int g = 0; g < Gd; ++g) {
            const uint2 sv = *reinterpret_cast<const uint2*>(Dm.s + mb + (size_t)g * H);
            const uint2 bv = *reinterpret_cast<const uint2*>(Dm.b + mb + (size_t)g * H);
            const uint32_t ws[4] = {sv.x << 16, sv.x & 0xffff0000u, sv.y << 16, sv.y & 0xffff0000u};
            const uint32_t wb[4] = {bv.x << 16, bv.x & 0xffff0000u, bv.y << 16, bv.y & 0xffff0000u};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                mx[j] = max(mx[j], ws[j] & 0x7fff0000u);
                mxb[j] = max(mxb[j], wb[j] & 0x7fff0000u);
            }
        }
        float ps[4], pb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int P = pf_row_pow2(mx[j], mxb[j]);
            ps[j] = ldexpf(1.0f, P);
            pb[j] = ldexpf(1.0f, P - 24);
            a.pdn[(size_t)slot * H + h + j] = ldexpf(1.0f, 24 - P);
        }
        for (int gp = 0; gp < GPd; ++gp) {
            uint32_t o[2][4];  // [group of the pair][row]; a missing second group (Gd odd) is zero
#pragma unroll
            for (int g2 = 0; g2 < 2; ++g2) {
                const int g = 2 * gp + g2;
                uint2 sv = make_uint2(0u, 0u), bv = make_uint2(0u, 0u);
                if (g < Gd) {
                    sv = *reinterpret_cast<const uint2*>(Dm.s + mb + (size_t)g * H);
                    bv = *reinterpret_cast<const uint2*>(Dm.b + mb + (size_t)g * H);
                }
                const uint32_t ws[4] = {sv.x << 16, sv.x & 0xffff0000u, sv.y << 16, sv.y & 0xffff0000u};
                const uint32_t wb[4] = {bv.x << 16, bv.x & 0xffff0000u, bv.y << 16, bv.y & 0xffff0000u};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[g2][j] = vmi_h2_bits((_Float16)(__uint_as_float(ws[j]) * ps[j]), (_Float16)(__uint_as_float(wb[j]) * pb[j]));
            }
            uint4* tp = reinterpret_cast<uint4*>(a.tdn + (((size_t)slot * GPd + gp) * H + h) * 2);
            tp[0] = make_uint4(o[0][0], o[1][0], o[0][1], o[1][1]);
            tp[1] = make_uint4(o[0][2], o[1][2], o[0][3], o[1][3]);
        }
    }
}

// Gate/up: tile 128 routes x 256 intermediate rows of gate and of up (512
// weight rows), K = H, eight waves side by side (wave w: all 128 routes,
// intermediate rows 32w.. of both matrices, so each dequantised weight
// operand feeds up to eight 16-route blocks).  The weight operand is the
// dequantised value in fp16, (q 2^-24) s' + b', with (s', b') from the table
// k_pf_table built (s' = s 2^P, b' = b 2^(P-24), P the row's power of two), so
// the MFMAs accumulate the whole affine product over all of K and the row's
// sums are times 2^(24-P) at the end.  K streams two quantisation groups per
// stage: the operand rows (gathered by token, shared by the waves: two slots
// and a barrier per stage) and each wave's own weight blocks and table pairs
// (two slots, no barrier: a wave DMAs exactly what it reads); the next
// group's weights are dequantised under the current group's MFMAs.  Then
// SwiGLU rounded to bf16, and the down projection's fp16 operands of the
// activations: each route's 256 columns times 2^-E, E the route's exponent for
// this block.
constexpr int kPf8Threads = 512;
constexpr int kPfA2 = kTM3 * 256;    // operand slot: 128 rows x two groups of 64 fp16
constexpr int kPfB2 = 8 * 4 * 1024;  // weight slot: per wave 4 pool blocks (16 rows x one group pair)
constexpr int kPfT2 = 8 * 512;       // table slot: per wave 64 rows x two groups x (s', b')
// byte offset of operand row r, logical 16-byte piece c (of 16), in a
// two-group slot: rows are 256 bytes (one pass over the 64 banks), so piece c
// sits at position c ^ (r & 15) and the 16 rows of a ds_read_b128 phase cover
// the banks once
__device__ __forceinline__ uint32_t pf_a2_off(int r, int c) { return 16u * (16u * r + (unsigned)(c ^ (r & 15))); }
// the logical piece a position holds (the inverse of pf_a2_off's swizzle)
__device__ __forceinline__ int pf_a2_piece(int r, int pos) { return pos ^ (r & 15); }

__global__ __launch_bounds__(kPf8Threads, 1) void k_pf_gateup3(PfArgs a) {
    // [operand slots 0, 1][weight slots 0, 1][table slots 0, 1]; after the
    // loop all of it holds the activation staging
    __shared__ __attribute__((aligned(16))) uint8_t s_mem[2 * (kPfA2 + kPfB2 + kPfT2)];
    uint8_t* const s_ra = s_mem;
    uint8_t* const s_rb = s_mem + 2 * kPfA2;
    uint8_t* const s_rt = s_rb + 2 * kPfB2;
    __shared__ __attribute__((aligned(16))) float s_post[512];  // 2^(24 - P): the row's sums are times this at the end
    __shared__ int s_route[kTM3];
    __shared__ int s_tok[kTM3];
    __shared__ float s_inv[kTM3];  // 1 / f of the route's token (0 past the tile)
    __shared__ int s_rexp[kTM3];   // E of each route row's activations
    const int tid = threadIdx.x, lane = tid & 63, w = pf_wave();
    const int n = lane & 15, q = lane >> 4;
    const int NB = (a.I + 255) / 256;
    int ti, nb;
    pf_tile_of(blockIdx.x, NB, ti, nb);
    if (ti >= a.ntiles[0]) return;
    const int4 tl = a.tiles[ti];
    const int H = a.H, HW = H / 8, G = H / 64, GP = G / 2, I = a.I;
    const int n0 = nb * 256, nvalid = min(256, I - n0);
    // 16-route blocks holding routes (uniform): the blocks past the tile's
    // count issue no MFMA
    const int mcnt = __builtin_amdgcn_readfirstlane(max(0, min(8, (tl.z + 15) / 16)));
    VMI_STAMP(4, 0);
    const vmi_qmat Gm = tl.x >= 0 ? a.gate : a.sh_gate;
    const vmi_qmat Um = tl.x >= 0 ? a.up : a.sh_up;
    const size_t mrow0 = (tl.x >= 0 ? (size_t)tl.x : 0) * (size_t)I;
    const int slot = tl.x >= 0 ? tl.x : a.cap;  // table slot (cap: the shared expert)
    // weight DMA of wave w: block b = 2mt + sb is pool block (rows n0 + 32w +
    // 16sb .. + 15 of matrix mt, group pair gp), 1 KB contiguous: 16 bytes of
    // group 2gp + g2, half h of row i at 16 (16 (2 g2 + h) + i).  Blocks past
    // I (a partial last column block) fetch the last block again.
    const uint32_t* bsrc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const int mt = b >> 1, sb = b & 1, rr = min(n0 + 32 * w + 16 * sb, I - 16);
        bsrc[b] = (mt ? Um.w : Gm.w) + mrow0 * HW + (size_t)(rr >> 4) * (H / 128) * 256 + 4 * lane;
    }
    // table DMA of wave w, per matrix: rows n0 + 32w + lane/2, group lane%2 of
    // the pair, one dword each
    const uint32_t* tsrc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const int row = min(n0 + 32 * w + (lane >> 1), I - 1);
        tsrc[mt] = a.tgu + (((size_t)slot * GP * 2 + mt) * I + row) * 2 + (lane & 1);
    }
    auto issue_b = [&](int gp, int u) {
        uint8_t* B = s_rb + u * kPfB2 + 4096 * w;
#pragma unroll
        for (int b = 0; b < 4; ++b) vmi_lds_dma16_opaque(bsrc[b] + 256 * gp, B + 1024 * b);
        uint8_t* Tt = s_rt + u * kPfT2 + 512 * w;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) vmi_lds_dma4_opaque(tsrc[mt] + (size_t)gp * 4 * I, Tt + 256 * mt);
    };
    // the first two group pairs' weights are in flight while the prologue runs
    issue_b(0, 0);
    issue_b(GP > 1 ? 1 : 0, 1);
    if (tid < kTM3) {
        const int rt = tile_route(a, tl, tid);
        const int tok = rt >= 0 ? rt / (a.k + 1) : 0;
        s_route[tid] = rt;
        s_tok[tid] = tok;
        s_inv[tid] = rt >= 0 ? 1.0f / a.fscale[tok] : 0.0f;
    }
    s_post[tid] = a.pgu[((size_t)slot * 2 + (tid >> 8)) * I + min(n0 + (tid & 255), I - 1)];
    __syncthreads();
    // operand DMA: pieces p = tid + 512 j (row p/16, position p%16 holding
    // logical piece pf_a2_piece(row, p%16) of the pair)
    const vmi_u4* asrc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = tid + kPf8Threads * j;
        const int arow = p >> 4, c = pf_a2_piece(arow, p & 15);
        asrc[j] = a.xop4 + (size_t)s_tok[arow] * HW + c;
    }
    auto issue_a = [&](int gp, int u) {
        uint8_t* A = s_ra + u * kPfA2;
#pragma unroll
        for (int j = 0; j < 4; ++j) vmi_lds_dma16_opaque(asrc[j] + 16 * gp, A + 16 * (kPf8Threads * j + 64 * w));
    };
    issue_a(0, 0);
    // this wave's four (column block, matrix) weight operands of group g2 of
    // the pair in slot u, dequantised
    auto dequant = [&](vmi_u4 (&bo)[4][2], int u, int g2) {
        const uint8_t* B = s_rb + u * kPfB2 + 4096 * w;
        const uint8_t* Tt = s_rt + u * kPfT2 + 512 * w;
#pragma unroll
        for (int blk = 0; blk < 4; ++blk) {
            const int sb = blk >> 1, mt = blk & 1;
            const uint2 wq = *reinterpret_cast<const uint2*>(B + 1024 * (2 * mt + sb) + 256 * (2 * g2 + (q >> 1)) +
                                                             16 * n + 8 * (q & 1));
            uint32_t s2, b2, b16;
            pf_affine_pairs(*reinterpret_cast<const uint32_t*>(Tt + 256 * mt + 4 * (2 * (16 * sb + n) + g2)), s2, b2, b16);
            bo[blk][0] = pf_dequant_f16(wq.x, s2, b2, b16);
            bo[blk][1] = pf_dequant_f16(wq.y, s2, b2, b16);
        }
    };
    vmi_f4 acc[8][2][2];
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int sb = 0; sb < 2; ++sb)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) acc[m][sb][mt] = vmi_f4{0.f, 0.f, 0.f, 0.f};
    VMI_STAMP(4, 1);
    // the stage loop for MC of the 16-route blocks holding routes (a loop per
    // MC, so each keeps its own register allocation; MC = 0 only moves the
    // rings and keeps the barriers).  Per thread and stage the DMA is 4
    // operand pieces and 6 weight and table copies, issued in the order the
    // waits below count.
    auto stage_loop = [&](auto mc_tag) {
        constexpr int MC = decltype(mc_tag)::value;
        // one group of the stage's pair: each 16-route block's operands (read
        // one block ahead) against the four weight operands; the weights go
        // first, so a lane holds four consecutive weight rows of one route
        auto mfma_group = [&](const uint8_t* A, int g2, const vmi_u4 (&bo)[4][2]) {
            vmi_u4 an0 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(n, 8 * g2 + 2 * q));
            vmi_u4 an1 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(n, 8 * g2 + 2 * q + 1));
#pragma unroll
            for (int m = 0; m < MC; ++m) {
                const vmi_u4 a0 = an0, a1 = an1;
                if (m + 1 < MC) {
                    const int row = 16 * (m + 1) + n;
                    an0 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(row, 8 * g2 + 2 * q));
                    an1 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(row, 8 * g2 + 2 * q + 1));
                }
#pragma unroll
                for (int blk = 0; blk < 4; ++blk)
                    acc[m][blk >> 1][blk & 1] = vmi_mfma_f16(bo[blk][0], a0, acc[m][blk >> 1][blk & 1]);
#pragma unroll
                for (int blk = 0; blk < 4; ++blk)
                    acc[m][blk >> 1][blk & 1] = vmi_mfma_f16(bo[blk][1], a1, acc[m][blk >> 1][blk & 1]);
            }
        };
        vmi_u4 b0[4][2], b1[4][2];  // group 0 and group 1 of a pair
        if constexpr (MC > 0) {
            pf_wait_vmcnt<4>();  // this wave's weights of pair 0 (operands 0 may be in flight)
            dequant(b0, 0, 0);
        }
#pragma unroll 1
        for (int gp = 0; gp < GP; ++gp) {
            const int u = gp & 1;
            // operands gp (this thread's pieces) have landed; weights gp + 1
            // may still be in flight
            if (gp == 0)
                pf_wait_vmcnt<0>();
            else
                pf_wait_vmcnt<6>();
            __syncthreads();  // everyone's operands gp; operand slot u ^ 1 is free
            if ((gp & 1) == 0 && gp < 16) VMI_STAMP(4, 2 + (gp >> 1));
            issue_a(min(gp + 1, GP - 1), u ^ 1);
            if constexpr (MC > 0) {
                dequant(b1, u, 1);
                mfma_group(s_ra + u * kPfA2, 0, b0);
            }
            // weight slot u is read: pair gp + 2 refills it (past the last
            // pair, the last again: never read)
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            issue_b(min(gp + 2, GP - 1), u);
            if constexpr (MC > 0) {
                pf_wait_vmcnt<10>();  // this wave's weights of pair gp + 1
                dequant(b0, u ^ 1, 0);  // past the last pair: stale values, unused
                mfma_group(s_ra + u * kPfA2, 1, b1);
            }
        }
    };
    switch (mcnt) {
        case 8: stage_loop(std::integral_constant<int, 8>{}); break;
        case 7: stage_loop(std::integral_constant<int, 7>{}); break;
        case 6: stage_loop(std::integral_constant<int, 6>{}); break;
        case 5: stage_loop(std::integral_constant<int, 5>{}); break;
        case 4: stage_loop(std::integral_constant<int, 4>{}); break;
        case 3: stage_loop(std::integral_constant<int, 3>{}); break;
        case 2: stage_loop(std::integral_constant<int, 2>{}); break;
        case 1: stage_loop(std::integral_constant<int, 1>{}); break;
        default: stage_loop(std::integral_constant<int, 0>{}); break;
    }
    pf_wait_vmcnt<0>();
    __syncthreads();
    VMI_STAMP(4, 10);
    // the rows' power-of-two factors out of the sums (exact): lane (n, q)
    // holds route row 16m + n, weight rows 256mt + 32w + 16sb + 4q .. + 3
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const float4 p4 = *reinterpret_cast<const float4*>(&s_post[256 * mt + 32 * w + 16 * sb + 4 * q]);
#pragma unroll
            for (int m = 0; m < 8; ++m) {
                acc[m][sb][mt][0] *= p4.x;
                acc[m][sb][mt][1] *= p4.y;
                acc[m][sb][mt][2] *= p4.z;
                acc[m][sb][mt][3] *= p4.w;
            }
        }
    __syncthreads();
    VMI_STAMP(4, 11);
    // SwiGLU into LDS as bf16 (the rounding of the activations):
    // route row 16m + n, columns 32w + 16sb + 4q .. + 3 (one 8-byte store);
    // the 16-route blocks past the tile's count hold no route
    constexpr int AS = 264;
    static_assert(kTM3 * AS * 2 <= sizeof(s_mem), "activation staging exceeds the ring and table");
    uint16_t* s_act = reinterpret_cast<uint16_t*>(s_mem);  // [128][AS]
#pragma unroll
    for (int m = 0; m < 8; ++m) {
        if (m >= mcnt) break;
        const int row = 16 * m + n;
        const float inv = s_inv[row];
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float gv = acc[m][sb][0][r] * inv, uv = acc[m][sb][1][r] * inv;
                // hardware exp2 and reciprocal (about 1 ulp each): the value is
                // rounded to bf16 right after
                const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-gv * 1.44269504f));
                v[r] = gv * sg * uv;
            }
            uint2 o;
            o.x = vmi_pack_bf16x2(v[0], v[1]);
            o.y = vmi_pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<uint2*>(s_act + row * AS + 32 * w + 16 * sb + 4 * q) = o;
        }
    }
    __syncthreads();
    VMI_STAMP(4, 13);
    // each route row's largest |activation| over the block's columns (four
    // lanes per row, 64 columns each; float bits ordered as integers) gives
    // its exponent E: the largest value times 2^-E lies in [2^14, 2^15).  E
    // is at least -40, so the down kernel's rescale 2^(E_prev - E) between
    // blocks stays finite (a block whose values are all below 2^-25 loses
    // what falls under fp16's subnormals)
    {
        const int row = tid >> 2, part = tid & 3;
        uint32_t mx = 0u;
        if (64 * part < nvalid) {
#pragma unroll
            for (int c = 0; c < 64; c += 8) {
                const vmi_u4 v = *reinterpret_cast<const vmi_u4*>(s_act + row * AS + 64 * part + c);
#pragma unroll
                for (int e = 0; e < 4; ++e) mx = max(mx, max((v[e] << 16) & 0x7fff0000u, v[e] & 0x7fff0000u));
            }
        }
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 1));
        mx = max(mx, (uint32_t)__shfl_xor((int)mx, 2));
        int e = 0;
        (void)frexpf(__uint_as_float(mx), &e);  // mx = f 2^e, f in [0.5, 1)
        if (part == 0) s_rexp[row] = mx ? max(e - 15, -40) : 0;
    }
    __syncthreads();
    const int IW = I / 8, IB = (I + 255) / 256, nw8 = nvalid / 8;
    for (int i = tid; i < kTM3 * nw8; i += kPf8Threads) {
        const int row = i / nw8, wd = i - row * nw8;
        const int route = s_route[row];
        if (route < 0) continue;
        const vmi_u4 v = *reinterpret_cast<const vmi_u4*>(s_act + row * AS + 8 * wd);
        const float fe = ldexpf(1.0f, -s_rexp[row]), fo = 0.0625f * fe;  // odd slots also divided by 16
        const uint32_t b0 = v[0] << 16, b1 = v[0] & 0xffff0000u, b2 = v[1] << 16, b3 = v[1] & 0xffff0000u;
        const uint32_t b4 = v[2] << 16, b5 = v[2] & 0xffff0000u, b6 = v[3] << 16, b7 = v[3] & 0xffff0000u;
        vmi_u4 o;  // slot order of vmi_unpack_u4_f16: {0,4,1,5,2,6,3,7}, exact (bf16 times a power of two)
        o[0] = vmi_h2_bits((_Float16)(__uint_as_float(b0) * fe), (_Float16)(__uint_as_float(b4) * fe));
        o[1] = vmi_h2_bits((_Float16)(__uint_as_float(b1) * fo), (_Float16)(__uint_as_float(b5) * fo));
        o[2] = vmi_h2_bits((_Float16)(__uint_as_float(b2) * fe), (_Float16)(__uint_as_float(b6) * fe));
        o[3] = vmi_h2_bits((_Float16)(__uint_as_float(b3) * fo), (_Float16)(__uint_as_float(b7) * fo));
        a.actop[(size_t)route * IW + (n0 >> 3) + wd] = o;
    }
    if (tid < kTM3 && s_route[tid] >= 0) a.aexp[(size_t)s_route[tid] * IB + nb] = s_rexp[tid];
    VMI_STAMP(4, 12);
}

// Down: tile 128 routes x 512 hidden rows, K = I, eight waves side by side
// (wave w: all 128 routes, hidden rows 64w..).  The MFMAs take the weights
// first, so a lane holds consecutive hidden rows of one route (y
// transposed); the weight rows of column blocks 2t and 2t + 1 interleave in
// fours (row 8i + r of the pair feeds MFMA row 4i + r of block 2t, row
// 8i + 4 + r that of block 2t + 1), so a lane's eight outputs of a pair are
// consecutive and one 16-byte store.  The weight operand is the dequantised
// value in fp16, (q 2^-24) s' + b' by one packed FMA per two values, with
// s' = s 2^P and b' = b 2^(P-24) for the hidden row's power of two P
// (pf_row_pow2); the activations are fp16 times 2^-E,
// E per route and 256-column block.  The sums are scaled by 2^(E_prev - E) at
// each block boundary and by 2^(24-P) 2^E_last at the end, then times the
// route's combine weight into one bf16 row per (token, rank).  As in
// k_pf_gateup3, K streams two groups per stage: the operand rows through two
// shared slots, each wave's own weight rows and table pairs through two slots
// of its own, dequantised one group ahead under the MFMAs.
constexpr int kPfMaxIB = 8;  // 256-column blocks of the intermediate size (I <= 2048)
// Hidden row (inside a wave's 64) of weight position p: positions 16sb..16sb+15
// are MFMA block sb's rows, and row n of block sb (= 2t + s) is hidden row
// 32t + 8(n/4) + 4s + n%4, so a lane's outputs of blocks 2t and 2t + 1 are
// eight consecutive hidden rows.
__device__ __forceinline__ int pf_down_row(int p) {
    return (p & 32) | (((p >> 2) & 3) << 3) | (((p >> 4) & 1) << 2) | (p & 3);
}

__global__ __launch_bounds__(kPf8Threads, 1) void k_pf_down3(PfArgs a) {
    // [operand slots 0, 1][weight slots 0, 1][table slots 0, 1], one group
    // pair each
    __shared__ __attribute__((aligned(16))) uint8_t s_mem[2 * (kPfA2 + kPfB2 + kPfT2)];
    uint8_t* const s_ra = s_mem;
    uint8_t* const s_rb = s_mem + 2 * kPfA2;
    uint8_t* const s_rt = s_rb + 2 * kPfB2;
    __shared__ __attribute__((aligned(16))) float s_post[2 * 512];  // 2^(24 - P) of the column blocks' rows
    __shared__ int s_route[kTM3];
    __shared__ int s_exp[kTM3][kPfMaxIB];
    __shared__ float s_rf[kTM3];  // the route's combine weight times 2^E of its last block
    const int tid = threadIdx.x, lane = tid & 63, w = pf_wave();
    const int n = lane & 15, q = lane >> 4;
    const int NBL = pf_down_blocks(a.H), NB = a.H / (512 * NBL);
    int ti, nb;
    pf_tile_of(blockIdx.x, NB, ti, nb);
    if (ti >= a.ntiles[0]) return;
    const int4 tl = a.tiles[ti];
    // 16-route blocks holding routes (uniform): the blocks past the tile's
    // count issue no MFMA
    const int mcnt = __builtin_amdgcn_readfirstlane(max(0, min(8, (tl.z + 15) / 16)));
    VMI_STAMP(3, 0);
    const int H = a.H, I = a.I, IW = I / 8, G = I / 64, GP = (G + 1) / 2, IB = (I + 255) / 256;
    const int h0 = nb * 512 * NBL;
    const vmi_qmat Dm = tl.x >= 0 ? a.down : a.sh_down;
    const int slot = tl.x >= 0 ? tl.x : a.cap;  // table slot (cap: the shared expert)
    // the down projection is group-major: row h of group g of slot m at
    // (m * G + g) * H + h (32 bytes of words)
    const size_t mbase = (tl.x >= 0 ? (size_t)tl.x : 0) * (size_t)G * H + h0 + 64 * w;
    // weight DMA into the wave's own 2 KB per group: 32-byte position
    // p = 32j + lane/2 holds hidden row 64w + pf_down_row(p), half
    // (lane%2) ^ bit 3 of p (pf_down_row puts the 16 rows an MFMA block reads
    // in 16 consecutive positions, which ds_read_b64 reads without bank
    // conflicts)
    const uint32_t* bsrc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int p = 32 * j + (lane >> 1), h = (lane & 1) ^ ((p >> 3) & 1);
        bsrc[j] = Dm.w + (mbase + pf_down_row(p)) * 8 + 4 * h;
    }
    // table DMA: the wave's 64 hidden rows in order, two words (the pair's
    // groups) each
    const uint32_t* tsrc = a.tdn + ((size_t)slot * GP * H + h0 + 64 * w) * 2 + lane;
    // pair v of the workgroup's sequence: column block v / GP, group pair v % GP
    auto issue_b = [&](int v, int u) {
        const int blk = v >= GP ? 1 : 0, gp = v - blk * GP;
        uint8_t* B = s_rb + u * kPfB2 + 4096 * w;
#pragma unroll
        for (int g2 = 0; g2 < 2; ++g2) {
            // a missing second group (G odd) fetches the last again: its table pair is zero
            const int g = min(2 * gp + g2, G - 1);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                vmi_lds_dma16_opaque(bsrc[j] + ((size_t)g * H + 512 * blk) * 8, B + 2048 * g2 + 1024 * j);
        }
        uint8_t* Tt = s_rt + u * kPfT2 + 512 * w;
#pragma unroll
        for (int j = 0; j < 2; ++j) vmi_lds_dma4_opaque(tsrc + ((size_t)gp * H + 512 * blk) * 2 + 64 * j, Tt + 256 * j);
    };
    // the first two pairs' weights are in flight while the prologue runs
    const int NV = NBL * GP;
    issue_b(0, 0);
    issue_b(NV > 1 ? 1 : 0, 1);
    if (tid < kTM3) {
        const int rt = tile_route(a, tl, tid);
        s_route[tid] = rt;
        int el = 0;
        for (int b = 0; b < IB; ++b) {
            el = rt >= 0 ? a.aexp[(size_t)rt * IB + b] : 0;
            s_exp[tid][b] = el;
        }
        float wgt = 0.0f;
        if (rt >= 0) {
            const int t = rt / (a.k + 1), j = rt - t * (a.k + 1);
            wgt = j < a.k ? a.scores[t * a.k + j] : (a.has_sgate ? 1.0f / (1.0f + expf(-a.sglogit[t])) : 1.0f);
        }
        s_rf[tid] = wgt * ldexpf(1.0f, el);
    }
    s_post[tid] = a.pdn[(size_t)slot * H + h0 + tid];
    if (NBL == 2) s_post[512 + tid] = a.pdn[(size_t)slot * H + h0 + 512 + tid];
    __syncthreads();
    // operand DMA: pieces p = tid + 512 j (row p/16, position p%16 holding
    // logical piece pf_a2_piece(row, p%16) of the pair); a missing second
    // group reads the first again (its weights are zero)
    const vmi_u4* asrc[4];
    int apc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = tid + kPf8Threads * j;
        const int arow = p >> 4;
        const int rt = s_route[arow];
        apc[j] = pf_a2_piece(arow, p & 15);
        asrc[j] = a.actop + (size_t)(rt >= 0 ? rt : 0) * IW;
    }
    auto issue_a = [&](int v, int u) {
        const int gp = v >= GP ? v - GP : v;
        uint8_t* A = s_ra + u * kPfA2;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int pc = 16 * gp + apc[j];
            vmi_lds_dma16_opaque(asrc[j] + (pc < IW ? pc : pc - 8), A + 16 * (kPf8Threads * j + 64 * w));
        }
    };
    issue_a(0, 0);
    // this wave's four column blocks of group g2 of the pair in slot u,
    // dequantised; block sb row n is hidden row 64w + pf_down_row(16sb + n)
    auto dequant = [&](vmi_u4 (&wo)[4][2], int u, int g2) {
        const uint8_t* B = s_rb + u * kPfB2 + 4096 * w + 2048 * g2;
        const uint8_t* Tt = s_rt + u * kPfT2 + 512 * w;
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            const int pos = 16 * sb + n;
            const uint2 wq = *reinterpret_cast<const uint2*>(B + ring_off(pos, q));
            uint32_t s2, b2, b16;
            pf_affine_pairs(*reinterpret_cast<const uint32_t*>(Tt + 4 * (2 * pf_down_row(pos) + g2)), s2, b2, b16);
            wo[sb][0] = pf_dequant_f16(wq.x, s2, b2, b16);
            wo[sb][1] = pf_dequant_f16(wq.y, s2, b2, b16);
        }
    };
    vmi_f4 acc[8][4];
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) acc[m][sb] = vmi_f4{0.f, 0.f, 0.f, 0.f};
    VMI_STAMP(3, 1);
    // the stage loop for MC active 16-route blocks (a loop per MC, so each
    // keeps its own register allocation; MC = 0 only moves the rings and
    // keeps the barriers).  Per thread and stage the DMA is 4 operand pieces
    // and 6 weight and table copies, issued in the order the waits count.
    auto stage_loop = [&](auto mc_tag) {
        constexpr int MC = decltype(mc_tag)::value;
        auto mfma_group = [&](const uint8_t* A, int g2, const vmi_u4 (&wo)[4][2]) {
            vmi_u4 an0 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(n, 8 * g2 + 2 * q));
            vmi_u4 an1 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(n, 8 * g2 + 2 * q + 1));
#pragma unroll
            for (int m = 0; m < MC; ++m) {
                const vmi_u4 a0 = an0, a1 = an1;
                if (m + 1 < MC) {
                    const int row = 16 * (m + 1) + n;
                    an0 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(row, 8 * g2 + 2 * q));
                    an1 = *reinterpret_cast<const vmi_u4*>(A + pf_a2_off(row, 8 * g2 + 2 * q + 1));
                }
#pragma unroll
                for (int sb = 0; sb < 4; ++sb) acc[m][sb] = vmi_mfma_f16(wo[sb][0], a0, acc[m][sb]);
#pragma unroll
                for (int sb = 0; sb < 4; ++sb) acc[m][sb] = vmi_mfma_f16(wo[sb][1], a1, acc[m][sb]);
            }
        };
        // column block blk's results: times 2^(24-P) of the row and the
        // route's weight, one bf16 row piece per lane (lane (n, q): route row
        // 16m + n, hidden rows 64w + 32t + 8q .. + 7 of the block), then the
        // sums start again
        auto store_block = [&](int blk) {
            float4 post[2][2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                post[t][0] = *reinterpret_cast<const float4*>(&s_post[512 * blk + 64 * w + 32 * t + 8 * q]);
                post[t][1] = *reinterpret_cast<const float4*>(&s_post[512 * blk + 64 * w + 32 * t + 8 * q + 4]);
            }
#pragma unroll
            for (int m = 0; m < MC; ++m) {
                const int route = s_route[16 * m + n];
                if (route >= 0) {
                    const float f = s_rf[16 * m + n];
                    uint16_t* yrow = a.ybuf + (size_t)route * H + h0 + 512 * blk + 64 * w + 8 * q;
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        const vmi_f4& lo = acc[m][2 * t];
                        const vmi_f4& hi = acc[m][2 * t + 1];
                        uint4 o;
                        o.x = vmi_pack_bf16x2(lo[0] * post[t][0].x * f, lo[1] * post[t][0].y * f);
                        o.y = vmi_pack_bf16x2(lo[2] * post[t][0].z * f, lo[3] * post[t][0].w * f);
                        o.z = vmi_pack_bf16x2(hi[0] * post[t][1].x * f, hi[1] * post[t][1].y * f);
                        o.w = vmi_pack_bf16x2(hi[2] * post[t][1].z * f, hi[3] * post[t][1].w * f);
                        *reinterpret_cast<uint4*>(yrow + 32 * t) = o;
                    }
                }
#pragma unroll
                for (int sb = 0; sb < 4; ++sb) acc[m][sb] = vmi_f4{0.f, 0.f, 0.f, 0.f};
            }
        };
        vmi_u4 b0[4][2], b1[4][2];  // group 0 and group 1 of a pair
        if constexpr (MC > 0) {
            pf_wait_vmcnt<4>();  // this wave's weights of pair 0 (operands 0 may be in flight)
            dequant(b0, 0, 0);
        }
        // a block's results are stored once every DMA issued so far has
        // landed (vmcnt 0), so the next pair needs no wait: the stores then
        // drain under its MFMAs instead of counting against its waits
        bool landed = false;
#pragma unroll 1
        for (int v = 0; v < NV; ++v) {
            const int u = v & 1;
            const int blk = v >= GP ? 1 : 0, gp = v - blk * GP;
            if (v == 0)
                pf_wait_vmcnt<0>();
            else if (!landed)
                pf_wait_vmcnt<6>();
            __syncthreads();  // everyone's operands v; operand slot u ^ 1 is free
            issue_a(min(v + 1, NV - 1), u ^ 1);
            if constexpr (MC > 0) {
                if (gp > 0 && (gp & 1) == 0) {
                    // a new 256-column block of K (two pairs): the sums so
                    // far times 2^(E_prev - E)
                    const int b = gp >> 1;
#pragma unroll
                    for (int m = 0; m < MC; ++m) {
                        const int row = 16 * m + n;
                        const float f = ldexpf(1.0f, s_exp[row][b - 1] - s_exp[row][b]);
#pragma unroll
                        for (int sb = 0; sb < 4; ++sb)
#pragma unroll
                            for (int r = 0; r < 4; ++r) acc[m][sb][r] *= f;
                    }
                }
                dequant(b1, u, 1);
                mfma_group(s_ra + u * kPfA2, 0, b0);
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): weight slot u is read
            issue_b(min(v + 2, NV - 1), u);
            if constexpr (MC > 0) {
                if (!landed) pf_wait_vmcnt<10>();  // this wave's weights of pair v + 1
                dequant(b0, u ^ 1, 0);  // past the last pair: stale values, unused
                mfma_group(s_ra + u * kPfA2, 1, b1);
            }
            landed = false;
            if (gp == GP - 1) {
                pf_wait_vmcnt<0>();
                if constexpr (MC > 0) store_block(blk);
                landed = true;
            }
        }
    };
    switch (mcnt) {
        case 8: stage_loop(std::integral_constant<int, 8>{}); break;
        case 7: stage_loop(std::integral_constant<int, 7>{}); break;
        case 6: stage_loop(std::integral_constant<int, 6>{}); break;
        case 5: stage_loop(std::integral_constant<int, 5>{}); break;
        case 4: stage_loop(std::integral_constant<int, 4>{}); break;
        case 3: stage_loop(std::integral_constant<int, 3>{}); break;
        case 2: stage_loop(std::integral_constant<int, 2>{}); break;
        case 1: stage_loop(std::integral_constant<int, 1>{}); break;
        default: stage_loop(std::integral_constant<int, 0>{}); break;
    }
    VMI_STAMP(3, 2);
    VMI_STAMP(3, 3);
    VMI_STAMP(3, 4);
}

// Router logits [T, E] as the same 128 x 128 tile GEMM (tokens x experts, K =
// H), dense: tile L/8-major as above with NB = 2 ceil(E/128) (expert block,
// half of K) pairs.  4-bit rows are 32 bytes a group (as gate/up); 8-bit rows
// 64 bytes, 16-byte piece c of row r kept at c ^ ((r >> 2) & 3).  Half kh of
// the logits = acc / f (+ bias in half 0); the top-k adds half 0 and half 1.
__device__ __forceinline__ uint32_t pf_b8_off(int r, int c) { return 16u * (4u * r + (unsigned)(c ^ ((r >> 2) & 3))); }

template <int BITS>
__global__ __launch_bounds__(kPfThreads, 2) void k_pf_router3(PfArgs a) {
    constexpr int kB = 128 * 8 * BITS;  // one group of 128 rows
    __shared__ __attribute__((aligned(16))) uint8_t s_ring[kPfStages * (kPfA + kB)];
    __shared__ uint16_t s_scale[kMaxG][128];
    const int tid = threadIdx.x, lane = tid & 63, w = pf_wave();
    const int n = lane & 15, q = lane >> 4;
    const int mh = w & 1, nh = w >> 1;
    // two workgroups per tile, one per half of K (kh), so a CU holds two
    const int NB = 2 * ((a.E + 127) / 128);
    int ti, nbk;
    pf_tile_of(blockIdx.x, NB, ti, nbk);
    const int t0 = ti * kTM3;
    if (t0 >= a.T) return;
    const int nb = nbk >> 1, kh = nbk & 1;
    const int H = a.H, HW = H / 8, G = H / 64, E = a.E;
    const int g0 = kh * (G / 2), g1 = g0 + G / 2;  // this half's groups
    const int e0 = nb * 128;
    const int wpr = H * BITS / 32;
    const vmi_u4* xop = a.xop4;  // the 8-bit words unpack into the same slot order
    const float* xsum = a.xsum4;
    for (int i = tid; i < 128 * (G / 8); i += kPfThreads) {
        const int chunk = i % (G / 8), row = i / (G / 8);
        const int e = min(e0 + row, E - 1);
        const uint4 v = *reinterpret_cast<const uint4*>(a.router.s + (size_t)e * G + 8 * chunk);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) s_scale[8 * chunk + j][row] = (uint16_t)((wv[j >> 1] >> (16 * (j & 1))) & 0xffffu);
    }
    __syncthreads();
    const vmi_u4* asrc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int p = tid + kPfThreads * j, row = p >> 3, c = pf_a_piece(row, p & 7);
        asrc[j] = xop + (size_t)min(t0 + row, a.T - 1) * HW + c;
    }
    constexpr int NBD = BITS == 8 ? 2 : 1;  // weight pieces per thread and group
    const uint32_t* bsrc[NBD];
#pragma unroll
    for (int j = 0; j < NBD; ++j) {
        const int p = tid + kPfThreads * j;
        int row, off;
        if constexpr (BITS == 8) {
            row = p >> 2;
            off = 4 * ((p & 3) ^ ((row >> 2) & 3));
        } else {
            row = p >> 1;
            off = 4 * ((p & 1) ^ ((row >> 3) & 1));
        }
        bsrc[j] = a.router.w + (size_t)min(e0 + row, E - 1) * wpr + off;
    }
    auto issue = [&](int g, int u) {
        uint8_t* A = s_ring + u * (kPfA + kB);
#pragma unroll
        for (int j = 0; j < 4; ++j) vmi_lds_dma16_opaque(asrc[j] + 8 * g, A + 16 * (kPfThreads * j + 64 * w));
#pragma unroll
        for (int j = 0; j < NBD; ++j)
            vmi_lds_dma16_opaque(bsrc[j] + 2 * BITS * g, A + kPfA + 16 * (kPfThreads * j + 64 * w));
    };
    vmi_f4 acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) acc[m][sb] = vmi_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kPfStages - 1; ++u) issue(g0 + u < g1 ? g0 + u : g1 - 1, u);
#pragma unroll 1
    for (int g = g0; g < g1; ++g) {
        const int u = (g - g0) % kPfStages;
        pf_wait_vmcnt<(4 + NBD) * (kPfStages - 2)>();
        __syncthreads();
        {
            const int gn = g + kPfStages - 1;
            issue(gn < g1 ? gn : g1 - 1, (gn - g0) % kPfStages);
        }
        const uint8_t* A = s_ring + u * (kPfA + kB);
        const uint8_t* B = A + kPfA;
        vmi_u4 av[4][2];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int row = 64 * mh + 16 * m + n;
            av[m][0] = *reinterpret_cast<const vmi_u4*>(A + pf_a_off(row, 2 * q));
            av[m][1] = *reinterpret_cast<const vmi_u4*>(A + pf_a_off(row, 2 * q + 1));
        }
        vmi_f4 dp[4];
        float scp = 0.0f;
#pragma unroll
        for (int sb = 0; sb <= 4; ++sb) {
            vmi_f4 dc[4];
            float scc = 0.0f;
            if (sb < 4) {
                const int brow = 64 * nh + 16 * sb + n;
                vmi_u4 b0, b1;
                if constexpr (BITS == 8) {
                    const uint4 ww = *reinterpret_cast<const uint4*>(B + pf_b8_off(brow, q));
                    b0 = unpack_u8_f16(ww.x, ww.y);
                    b1 = unpack_u8_f16(ww.z, ww.w);
                } else {
                    const uint2 ww = *reinterpret_cast<const uint2*>(B + ring_off(brow, q));
                    b0 = vmi_unpack_u4_f16(ww.x);
                    b1 = vmi_unpack_u4_f16(ww.y);
                }
                scc = vmi_bf16_to_f32(s_scale[g][brow]) * 16777216.0f;
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    dc[m] = vmi_mfma_f16(av[m][0], b0, vmi_f4{0.f, 0.f, 0.f, 0.f});
                    dc[m] = vmi_mfma_f16(av[m][1], b1, dc[m]);
                }
            }
            if (sb > 0) {
#pragma unroll
                for (int m = 0; m < 4; ++m)
#pragma unroll
                    for (int r = 0; r < 4; ++r) acc[m][sb - 1][r] = fmaf(dp[m][r], scp, acc[m][sb - 1][r]);
            }
            if (sb < 4) {
#pragma unroll
                for (int m = 0; m < 4; ++m) dp[m] = dc[m];
                scp = scc;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    pf_wait_vmcnt<0>();
    __syncthreads();
    // affine-bias term through bf16 MFMAs, as in k_pf_gateup3
    constexpr int XS = kMaxG + 1, BS = kMaxG / 2 + 1;
    static_assert(kTM3 * XS * 4 + 128 * BS * 4 <= sizeof(s_ring), "bias operands exceed the ring");
    float* s_xs = reinterpret_cast<float*>(s_ring);
    uint32_t* s_b = reinterpret_cast<uint32_t*>(s_ring + kTM3 * XS * 4);
    for (int i = tid; i < kTM3 * G; i += kPfThreads) {
        const int row = i / G, g = i - row * G;
        s_xs[row * XS + g] = xsum[(size_t)min(t0 + row, a.T - 1) * G + g];
    }
    for (int i = tid; i < 128 * (G / 2); i += kPfThreads) {
        const int row = i / (G / 2), c = i - row * (G / 2);
        s_b[row * BS + c] = reinterpret_cast<const uint32_t*>(a.router.b + (size_t)min(e0 + row, E - 1) * G)[c];
    }
    __syncthreads();
    // the affine terms of eight groups per MFMA: chunks [0, C/2) in the first
    // half's workgroup (rounded up), the rest in the second's
    const int C = G / 8, ch = (C + 1) / 2;
#pragma unroll 1
    for (int c8 = kh ? ch : 0; c8 < (kh ? C : ch); ++c8) {
        const int gq = 8 * c8 + 2 * q;
        vmi_u4 ab[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int row = 64 * mh + 16 * m + n;
            ab[m] = vmi_bias_a_operand(s_xs[row * XS + gq], s_xs[row * XS + gq + 1]);
        }
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            const int brow = 64 * nh + 16 * sb + n;
            const vmi_u4 bb = vmi_bias_b_operand(s_b[brow * BS + (gq >> 1)]);
#pragma unroll
            for (int m = 0; m < 4; ++m) acc[m][sb] = vmi_mfma_bf16(ab[m], bb, acc[m][sb]);
        }
    }
    float* const lo = a.logits + (size_t)kh * a.T * E;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = t0 + 64 * mh + 16 * m + 4 * q + r;
            if (t >= a.T) continue;
            const float inv = 1.0f / a.fscale[t];
#pragma unroll
            for (int sb = 0; sb < 4; ++sb) {
                const int e = e0 + 64 * nh + 16 * sb + n;
                if (e >= E) continue;
                float v = acc[m][sb][r] * inv;
                if (a.logit_bias && kh == 0) v += a.logit_bias[e];
                lo[(size_t)t * E + e] = v;
            }
        }
}

// --------------------------------------------------------------- combine
// out[t][h] = bf16(sum_{j <= k} y[t(k+1)+j][h] (valid routes, rank order) + residual)
__global__ __launch_bounds__(kPfThreads) void k_pf_combine(PfArgs a) {
    // one token per workgroup, 8 columns per thread and pass; every rank's
    // 16-byte piece is requested before the sums, which add the ranks in
    // order and then the residual, per column
    const int t = blockIdx.x;
    const int K1 = a.k + 1;
    uint32_t okm = 0u;  // ranks that contribute (uniform)
    for (int j = 0; j < K1; ++j) {
        const bool ok = j < a.k ? a.slots[t * a.k + j] >= 0 : a.has_shared != 0;
        okm |= (ok ? 1u : 0u) << j;
    }
    const vmi_u4 z4 = {0u, 0u, 0u, 0u};
    // the token's K1 rows are one contiguous run of ybuf, read once:
    // nontemporal, branch-free buffer loads (an absent rank reads as zero)
    const __amdgpu_buffer_rsrc_t ry = vmi_rsrc(a.ybuf + (size_t)t * K1 * a.H, (uint32_t)(K1 * a.H * 2));
    for (int h = threadIdx.x * 8; h < a.H; h += kPfThreads * 8) {
        vmi_u4 y[kPfMaxK + 1];
#pragma unroll
        for (int j = 0; j <= kPfMaxK; ++j)
            y[j] = j < K1 ? vmi_bload_b128_nt(ry, ((okm >> j) & 1u) ? (uint32_t)((j * a.H + h) * 2) : VMI_OOB, 0) : z4;
        const vmi_u4 rv = a.residual ? *reinterpret_cast<const vmi_u4*>(a.residual + (size_t)t * a.H + h) : z4;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j <= kPfMaxK; ++j) {
            if (j < K1 && ((okm >> j) & 1u)) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[2 * e] += __uint_as_float(y[j][e] << 16);
                    acc[2 * e + 1] += __uint_as_float(y[j][e] & 0xffff0000u);
                }
            }
        }
        if (a.residual) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[2 * e] += __uint_as_float(rv[e] << 16);
                acc[2 * e + 1] += __uint_as_float(rv[e] & 0xffff0000u);
            }
        }
        vmi_u4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = vmi_pack_bf16x2(acc[2 * e], acc[2 * e + 1]);
        *reinterpret_cast<vmi_u4*>(a.out + (size_t)t * a.H + h) = o;
    }
}

// -------------------------------------------------------------- workspace
struct PfLayout {
    size_t status, xop4, xsum4, fscale, logits, sglogit, ids, scores, slots, counts, fill,
        tiles, ntiles, list, tgu, pgu, tdn, pdn, actop, aexp, ybuf, bytes;
    int max_tiles;
};

// The dequantisation tables (k_pf_table), in the workspace or in a caller's
// buffer (vmi_moe_prefill_tables): gate/up pairs, gate/up factors, down pairs,
// down factors, each 256-byte aligned.
struct PfTables {
    size_t tgu, pgu, tdn, pdn, bytes;
};

PfTables pf_tables_layout(int H, int I, int cap) {
    PfTables L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += vmi::align256(bytes);
        return o;
    };
    L.tgu = take((size_t)(cap + 1) * (H / 128) * 2 * I * 2 * 4);
    L.pgu = take((size_t)(cap + 1) * 2 * I * 4);
    L.tdn = take((size_t)(cap + 1) * ((I / 64 + 1) / 2) * H * 2 * 4);
    L.pdn = take((size_t)(cap + 1) * H * 4);
    L.bytes = off;
    return L;
}

PfLayout pf_layout(int T, int k, int H, int I, int E, int cap, int router_bits) {
    PfLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += vmi::align256(bytes);
        return o;
    };
    const size_t R = (size_t)T * (k + 1);
    L.max_tiles = (T * k + kTM3 - 1) / kTM3 + cap + (T + kTM3 - 1) / kTM3;
    L.status = take(256);
    L.xop4 = take((size_t)T * (H / 8) * 16);
    L.xsum4 = take((size_t)T * (H / 64) * 4);  // the router's affine term
    L.fscale = take((size_t)T * 4);
    L.logits = take((size_t)2 * T * E * 4);
    L.sglogit = take((size_t)T * 4);
    L.ids = take((size_t)T * k * 4);
    L.scores = take((size_t)T * k * 4);
    L.slots = take((size_t)T * k * 4);
    L.counts = take((size_t)cap * 4);
    L.fill = take((size_t)T * k * 4);
    L.tiles = take((size_t)L.max_tiles * 16);
    L.ntiles = take(4);
    L.list = take((size_t)T * k * 4);
    const PfTables TB = pf_tables_layout(H, I, cap);
    const size_t tb = take(TB.bytes);
    L.tgu = tb + TB.tgu;
    L.pgu = tb + TB.pgu;
    L.tdn = tb + TB.tdn;
    L.pdn = tb + TB.pdn;
    L.actop = take(R * (I / 8) * 16);
    L.aexp = take(R * ((I + 255) / 256) * 4);
    L.ybuf = take(R * H * 2);
    L.bytes = off;
    return L;
}

}  // namespace

extern "C" size_t vmi_moe_prefill_workspace_bytes(int T, int top_k, int hidden, int inter, int num_experts, int cap,
                                                  int router_bits) {
    if (T <= 0 || top_k <= 0 || hidden <= 0 || inter <= 0 || num_experts <= 0 || cap <= 0) return 0;
    return pf_layout(T, top_k, hidden, inter, num_experts, cap, router_bits).bytes;
}

extern "C" int vmi_moe_prefill(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* residual,
                               uint16_t* out, int32_t* ids_out, float* scores_out, void* workspace,
                               size_t workspace_bytes, void* stream) {
    vmi::clear_error();
    if (!desc) return vmi::fail(VMI_ERR_INVALID, "null desc");
    const vmi_moe_layer_desc& D = *desc;
    if (T <= 0 || T > 65536) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d must be in [1, 65536]", T);
    if (D.bits != 4 || D.group != 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "bits=%d group=%d", D.bits, D.group);
    if (D.hidden != 512 && D.hidden != 1024 && D.hidden != 2048)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d must be 512, 1024 or 2048", D.hidden);
    if (D.inter % 64 || D.inter <= 0 || D.inter > 2048)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "inter=%d must be a multiple of 64 up to 2048", D.inter);
    if (D.num_experts % 64 || D.num_experts <= 0 || D.num_experts > kPfMaxE)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "num_experts=%d must be a multiple of 64 up to %d", D.num_experts,
                         kPfMaxE);
    if (D.top_k <= 0 || D.top_k > kPfMaxK || D.top_k > D.num_experts)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "top_k=%d", D.top_k);
    if (D.cap <= 0 || D.cap > 1024) return vmi::fail(VMI_ERR_UNSUPPORTED, "cap=%d must be in [1, 1024]", D.cap);
    if (D.router_bits != 4 && D.router_bits != 8) return vmi::fail(VMI_ERR_UNSUPPORTED, "router_bits=%d", D.router_bits);
    const bool has_shared = D.shared_gate.w != nullptr;
    const bool has_sgate = has_shared && D.shared_expert_gate.w != nullptr;
    if (has_sgate && D.shared_expert_gate_bits != 4 && D.shared_expert_gate_bits != 8)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "shared_expert_gate_bits=%d", D.shared_expert_gate_bits);
    if (!x || !out || !D.router.w || !D.gate.w || !D.up.w || !D.down.w)
        return vmi::fail(VMI_ERR_INVALID, "null x/out/weights");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(residual) |
         reinterpret_cast<uintptr_t>(D.router.w) | reinterpret_cast<uintptr_t>(D.gate.w) |
         reinterpret_cast<uintptr_t>(D.up.w) | reinterpret_cast<uintptr_t>(D.down.w) |
         reinterpret_cast<uintptr_t>(D.norm_weight)) & 15)
        return vmi::fail(VMI_ERR_INVALID, "x, out, residual, norm weight and packed weights must be 16-byte aligned");
    {
        // the GEMMs read scales and biases as 16-byte vectors
        uintptr_t sb = reinterpret_cast<uintptr_t>(D.router.s) | reinterpret_cast<uintptr_t>(D.router.b) |
                       reinterpret_cast<uintptr_t>(D.gate.s) | reinterpret_cast<uintptr_t>(D.gate.b) |
                       reinterpret_cast<uintptr_t>(D.up.s) | reinterpret_cast<uintptr_t>(D.up.b) |
                       reinterpret_cast<uintptr_t>(D.down.s) | reinterpret_cast<uintptr_t>(D.down.b);
        if (has_shared)
            sb |= reinterpret_cast<uintptr_t>(D.shared_gate.s) | reinterpret_cast<uintptr_t>(D.shared_gate.b) |
                  reinterpret_cast<uintptr_t>(D.shared_up.s) | reinterpret_cast<uintptr_t>(D.shared_up.b) |
                  reinterpret_cast<uintptr_t>(D.shared_down.s) | reinterpret_cast<uintptr_t>(D.shared_down.b);
        if (sb & 15) return vmi::fail(VMI_ERR_INVALID, "scales and biases must be 16-byte aligned");
    }
    if (reinterpret_cast<uintptr_t>(D.prefill_tables) & 15)
        return vmi::fail(VMI_ERR_INVALID, "prefill tables must be 16-byte aligned");
    const PfLayout L = pf_layout(T, D.top_k, D.hidden, D.inter, D.num_experts, D.cap, D.router_bits);
    if (!workspace || workspace_bytes < L.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", L.bytes, workspace_bytes);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    PfArgs a{};
    a.T = T; a.H = D.hidden; a.I = D.inter; a.E = D.num_experts; a.k = D.top_k; a.cap = D.cap;
    a.norm_topk = D.norm_topk_prob; a.router_bits = D.router_bits; a.sg_bits = D.shared_expert_gate_bits;
    a.has_shared = has_shared; a.has_sgate = has_sgate;
    a.x = x; a.norm_w = D.norm_weight; a.eps = D.norm_eps; a.residual = residual;
    a.router = D.router; a.logit_bias = D.router_logit_bias; a.table = D.slot_table;
    a.gate = D.gate; a.up = D.up; a.down = D.down;
    a.sh_gate = has_shared ? D.shared_gate : D.gate;
    a.sh_up = has_shared ? D.shared_up : D.up;
    a.sh_down = has_shared ? D.shared_down : D.down;
    a.sgate = D.shared_expert_gate;
    a.status = reinterpret_cast<uint32_t*>(ws + L.status);
    a.xop4 = reinterpret_cast<vmi_u4*>(ws + L.xop4);
    a.xsum4 = reinterpret_cast<float*>(ws + L.xsum4);
    a.fscale = reinterpret_cast<float*>(ws + L.fscale);
    a.logits = reinterpret_cast<float*>(ws + L.logits);
    a.sglogit = reinterpret_cast<float*>(ws + L.sglogit);
    a.ids = reinterpret_cast<int32_t*>(ws + L.ids);
    a.scores = reinterpret_cast<float*>(ws + L.scores);
    a.slots = reinterpret_cast<int32_t*>(ws + L.slots);
    a.counts = reinterpret_cast<int32_t*>(ws + L.counts);
    a.fill = reinterpret_cast<int32_t*>(ws + L.fill);
    a.tiles = reinterpret_cast<int4*>(ws + L.tiles);
    a.ntiles = reinterpret_cast<int32_t*>(ws + L.ntiles);
    a.list = reinterpret_cast<int32_t*>(ws + L.list);
    if (D.prefill_tables) {
        const PfTables TB = pf_tables_layout(D.hidden, D.inter, D.cap);
        uint8_t* tb = static_cast<uint8_t*>(const_cast<void*>(D.prefill_tables));
        a.tgu = reinterpret_cast<uint32_t*>(tb + TB.tgu);
        a.pgu = reinterpret_cast<float*>(tb + TB.pgu);
        a.tdn = reinterpret_cast<uint32_t*>(tb + TB.tdn);
        a.pdn = reinterpret_cast<float*>(tb + TB.pdn);
    } else {
        a.tgu = reinterpret_cast<uint32_t*>(ws + L.tgu);
        a.pgu = reinterpret_cast<float*>(ws + L.pgu);
        a.tdn = reinterpret_cast<uint32_t*>(ws + L.tdn);
        a.pdn = reinterpret_cast<float*>(ws + L.pdn);
    }
    a.actop = reinterpret_cast<vmi_u4*>(ws + L.actop);
    a.aexp = reinterpret_cast<int32_t*>(ws + L.aexp);
    a.ybuf = reinterpret_cast<uint16_t*>(ws + L.ybuf);
    a.out = out; a.ids_out = ids_out; a.scores_out = scores_out;
    a.max_tiles = L.max_tiles;

    hipStream_t s = static_cast<hipStream_t>(stream);
    const int tok_blocks = (T + 3) / 4;
    switch (D.hidden / 512) {
        case 1: hipLaunchKernelGGL(k_pf_prep<1>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a); break;
        case 2: hipLaunchKernelGGL(k_pf_prep<2>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a); break;
        case 4: hipLaunchKernelGGL(k_pf_prep<4>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a); break;
        default: return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d must be 512, 1024 or 2048", D.hidden);
    }
    const dim3 rgrid(8 * (((T + kTM3 - 1) / kTM3 + 7) / 8) * 2 * ((D.num_experts + 127) / 128));
    if (D.router_bits == 4)
        hipLaunchKernelGGL(k_pf_router3<4>, rgrid, dim3(kPfThreads), 0, s, a);
    else
        hipLaunchKernelGGL(k_pf_router3<8>, rgrid, dim3(kPfThreads), 0, s, a);
    {
        const int ni = D.num_experts / 64;  // key slots per lane, padded to a power of two
        if (ni <= 1)
            hipLaunchKernelGGL(k_pf_topk<1>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a);
        else if (ni <= 2)
            hipLaunchKernelGGL(k_pf_topk<2>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a);
        else if (ni <= 4)
            hipLaunchKernelGGL(k_pf_topk<4>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a);
        else if (ni <= 8)
            hipLaunchKernelGGL(k_pf_topk<8>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a);
        else
            hipLaunchKernelGGL(k_pf_topk<16>, dim3(tok_blocks), dim3(kPfThreads), 0, s, a);
    }
    hipLaunchKernelGGL(k_pf_count, dim3((T * D.top_k + kCountRoutes - 1) / kCountRoutes), dim3(kPfThreads), 0, s, a);
    hipLaunchKernelGGL(k_pf_place, dim3((T * D.top_k + kPfThreads - 1) / kPfThreads), dim3(kPfThreads), 0, s, a);
    if (!D.prefill_tables)
        hipLaunchKernelGGL(k_pf_table, dim3((D.cap + 1) * pf_table_blocks(D.hidden, D.inter)), dim3(kPfThreads), 0, s,
                           a);
    const int tile_slots = 8 * ((L.max_tiles + 7) / 8);
    hipLaunchKernelGGL(k_pf_gateup3, dim3(tile_slots * ((D.inter + 255) / 256)), dim3(kPf8Threads), 0, s, a);
    hipLaunchKernelGGL(k_pf_down3, dim3(tile_slots * (D.hidden / (512 * pf_down_blocks(D.hidden)))), dim3(kPf8Threads),
                       0, s, a);
    hipLaunchKernelGGL(k_pf_combine, dim3(T), dim3(kPfThreads), 0, s, a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "prefill launch");
}

extern "C" size_t vmi_moe_prefill_tables_bytes(int hidden, int inter, int cap) {
    if (hidden <= 0 || hidden % 512 || inter <= 0 || inter % 64 || cap <= 0) return 0;
    return pf_tables_layout(hidden, inter, cap).bytes;
}

extern "C" int vmi_moe_prefill_tables(const vmi_moe_layer_desc* desc, void* tables, size_t bytes, void* stream) {
    vmi::clear_error();
    if (!desc) return vmi::fail(VMI_ERR_INVALID, "null desc");
    const vmi_moe_layer_desc& D = *desc;
    if (D.bits != 4 || D.group != 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "bits=%d group=%d", D.bits, D.group);
    if (D.hidden != 512 && D.hidden != 1024 && D.hidden != 2048)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d must be 512, 1024 or 2048", D.hidden);
    if (D.inter % 64 || D.inter <= 0 || D.inter > 2048)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "inter=%d must be a multiple of 64 up to 2048", D.inter);
    if (D.cap <= 0 || D.cap > 1024) return vmi::fail(VMI_ERR_UNSUPPORTED, "cap=%d must be in [1, 1024]", D.cap);
    const bool has_shared = D.shared_gate.w != nullptr;
    if (!D.gate.s || !D.gate.b || !D.up.s || !D.up.b || !D.down.s || !D.down.b)
        return vmi::fail(VMI_ERR_INVALID, "null scales or biases");
    if (has_shared && (!D.shared_gate.s || !D.shared_gate.b || !D.shared_up.s || !D.shared_up.b ||
                       !D.shared_down.s || !D.shared_down.b))
        return vmi::fail(VMI_ERR_INVALID, "null shared-expert scales or biases");
    uintptr_t sb = reinterpret_cast<uintptr_t>(D.gate.s) | reinterpret_cast<uintptr_t>(D.gate.b) |
                   reinterpret_cast<uintptr_t>(D.up.s) | reinterpret_cast<uintptr_t>(D.up.b) |
                   reinterpret_cast<uintptr_t>(D.down.s) | reinterpret_cast<uintptr_t>(D.down.b);
    if (has_shared)
        sb |= reinterpret_cast<uintptr_t>(D.shared_gate.s) | reinterpret_cast<uintptr_t>(D.shared_gate.b) |
              reinterpret_cast<uintptr_t>(D.shared_up.s) | reinterpret_cast<uintptr_t>(D.shared_up.b) |
              reinterpret_cast<uintptr_t>(D.shared_down.s) | reinterpret_cast<uintptr_t>(D.shared_down.b);
    if (sb & 15) return vmi::fail(VMI_ERR_INVALID, "scales and biases must be 16-byte aligned");
    const PfTables TB = pf_tables_layout(D.hidden, D.inter, D.cap);
    if (!tables || bytes < TB.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "tables need %zu bytes (got %zu)", TB.bytes, bytes);
    if (reinterpret_cast<uintptr_t>(tables) & 15) return vmi::fail(VMI_ERR_INVALID, "tables must be 16-byte aligned");
    uint8_t* tb = static_cast<uint8_t*>(tables);
    PfArgs a{};
    a.H = D.hidden; a.I = D.inter; a.cap = D.cap; a.has_shared = has_shared;
    a.gate = D.gate; a.up = D.up; a.down = D.down;
    a.sh_gate = has_shared ? D.shared_gate : D.gate;
    a.sh_up = has_shared ? D.shared_up : D.up;
    a.sh_down = has_shared ? D.shared_down : D.down;
    a.counts = nullptr;  // every slot
    a.tgu = reinterpret_cast<uint32_t*>(tb + TB.tgu);
    a.pgu = reinterpret_cast<float*>(tb + TB.pgu);
    a.tdn = reinterpret_cast<uint32_t*>(tb + TB.tdn);
    a.pdn = reinterpret_cast<float*>(tb + TB.pdn);
    hipLaunchKernelGGL(k_pf_table, dim3((D.cap + 1) * pf_table_blocks(D.hidden, D.inter)), dim3(kPfThreads), 0,
                       static_cast<hipStream_t>(stream), a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "prefill tables launch");
}

#ifdef VMI_TIMELINE
extern "C" int vmi_timeline_set_prefill(unsigned long long* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(vmi_tl_buf), &buf, sizeof(buf)) == hipSuccess ? 0 : -1;
}
#endif
