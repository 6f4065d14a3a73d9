// Gated DeltaNet (linear attention) block of a Qwen3-Next decoder layer on a
// verify batch, with the recurrent state captured after every token.
//
// The reference runs this block through mlx-lm's Qwen3NextGatedDeltaNet; at
// verify time it is patched to capture, per token, the conv window and the
// recurrent state (mlx_streaming/mtp/kv_cache.py:34-102, multistate kernel
// core/linear_attn/gated_delta_multistate.py:27-143), so that committing an
// accepted prefix is selecting checkpoint accepted_len - 1
// (kv_cache.py:222-251).  Here both states live in rings indexed by absolute
// position, and committing is setting the cache length:
//   conv ring   bf16 [32][conv_dim]: row p % 32 holds the conv input of
//               position p (the projected [q | k | v] row); the window of
//               position p is positions p-3..p (zeros before position 0);
//   state ring  f32 [n_slots][n_v][dv][dk]: slot p % n_slots holds the state
//               after positions 0..p-1 (before position 0: zeros, not read).
// A batch at positions pos0..pos0+T-1 reads conv rows < pos0 and state slot
// pos0 % n_slots, and writes conv rows pos0.. and state slots pos0+1.. ; with
// n_slots >= T + 1 no slot it reads is overwritten.
//
// Kernels:
//   k_qgemv4 (vmi_attn.hip)  input RMSNorm and the qkvz and ba projections
//   k_gdn_block   per v-head: causal conv of width 4 + SiLU (conv input rows
//                 rounded to bf16 and appended to the ring), q/k normalisation,
//                 gate scalars, the delta rule over the T tokens in fp32 (state
//                 after each token to the ring), gated RMSNorm
//   k_qgemv4      out_proj with the residual add

#include "vmi_device.h"
#include "vmi_internal.h"

namespace {

constexpr int kGHead = 128;        // head_k_dim = head_v_dim
constexpr int kConvRing = 32;      // conv ring rows
constexpr int kConvTaps = 4;
constexpr int kGdnMaxT = 16;      // tokens of one call (a chain, or the paths of a tree)
constexpr int kGdnMaxSpan = 8;    // tokens of one path

// Floats per token of tree_side: k of every key head, v of every value head,
// then (g, beta) of every value head.
__host__ __device__ constexpr int vmi_gdn_tree_side_stride(int n_k, int n_v) {
    return n_k * kGHead + n_v * kGHead + 2 * n_v;
}

__device__ __forceinline__ int g_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

struct GdnArgs {
    int T, pos0, n_k, n_v, r;      // r = n_v / n_k
    int paths, span;               // T = paths * span: path p's tokens p*span .. at positions pos0 ..
    uint16_t* tree_conv;           // or null: [T][conv_dim] conv inputs instead of the ring
    float* tree_side;              // or null: [T][side_stride] k | v | (g, beta) instead of the states
    int side_stride;               // n_k * 128 + n_v * 128 + 2 * n_v
    const int32_t* pos_dev;        // if set: pos0 is read here (graph replays)
    int per_g, conv_dim, stride;   // proj row: [n_k groups of per_g | ba (2 n_v)]
    const float* proj;             // [T, stride] f32
    const uint16_t* conv_w;        // [conv_dim][4] bf16
    const float* A_log;            // [n_v]
    const float* dt_bias;          // [n_v]
    uint16_t* conv_ring;           // [32][conv_dim]
    float* state_ring;             // [n_slots][n_v][128][128]
    int n_slots;
    const uint16_t* norm_w;        // [128]
    float eps;
    uint16_t* o;                   // [T][n_v * 128] bf16
};

// Projection column of conv channel c (0 <= c < conv_dim).
__device__ __forceinline__ int conv_src(const GdnArgs& a, int c) {
    const int nq = a.n_k * kGHead;
    if (c < nq) return (c / kGHead) * a.per_g + (c % kGHead);
    if (c < 2 * nq) return ((c - nq) / kGHead) * a.per_g + kGHead + (c % kGHead);
    const int h = (c - 2 * nq) / kGHead;
    return (h / a.r) * a.per_g + 2 * kGHead + (h % a.r) * kGHead + (c % kGHead);
}

__device__ __forceinline__ int gdn_pos0(const GdnArgs& a) { return a.pos_dev ? max(*a.pos_dev, 0) : a.pos0; }

__device__ __forceinline__ float bf16_round(float f) { return vmi_bf16_to_f32(vmi_f32_to_bf16(f)); }

// One token of the delta rule on one state row held as 8 dk values per lane
// (16 lanes per row): S <- g S; delta = beta (v - S k); S <- S + delta k^T.
// The sum over dk is the DPP row reduction, so the result does not depend on
// which kernel applies the token.
__device__ __forceinline__ void gdn_row_update(float (&Sr)[8], const float (&kk)[8], float vv, float g, float beta) {
    float kv = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        Sr[i] *= g;
        kv = fmaf(Sr[i], kk[i], kv);
    }
    kv = vmi_row_sum16(kv);
    const float delta = (vv - kv) * beta;
#pragma unroll
    for (int i = 0; i < 8; ++i) Sr[i] = fmaf(kk[i], delta, Sr[i]);
}

// One workgroup of 1024 threads per v-head h (key head hk = h / r), the
// whole block between the projections in one launch:
//  1. the conv operands are requested first, then the state rows of the head
//     (thread: rows tid/16 and tid/16 + 64, dk 4 (tid % 16) .. + 3 and 64 +
//     the same, so that 16 lanes store 256 contiguous bytes of a row): loads
//     complete in issue order, so the conv waits for its own operands only
//     and the state arrives during 2-3;
//  2. conv: thread c < 384 owns channel c of [q(hk) | k(hk) | v(h)]: token
//     j of a path sees positions pos0+j-3 .. pos0+j (ring rows before pos0,
//     zeros before position 0, the path's projections rounded to bf16), the
//     causal conv of width 4 and SiLU per token into LDS; the batch rows go
//     to the conv ring, or for a tree to tree_conv (q/k channels by the first
//     v-head of the group only); threads 384.. the gate scalars
//     beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt_bias));
//  3. wave 2t + j normalises q (j = 0) or k (j = 1) of token t:
//     rms_norm(., 1e-6) / dk for q, / sqrt(dk) for k (lane l owns channels l
//     and l + 64, the canonical wave sum);
//  4. the delta rule over each path's tokens in fp32 from the state before
//     pos0, 16 lanes per state row (sums over dk by the DPP row reduction, the
//     same for every batch size, so a T-token call equals T one-token calls
//     bit for bit); the state after each token to the ring, the head output y
//     to LDS.  A tree stores no state: each token's k, v, g and beta go to
//     tree_side, from which the commit replays the winning path's tokens;
//  5. wave t: the gated RMSNorm of token t, y / rms * w * silu(z), to bf16.
constexpr int kGFThreads = 1024;
constexpr int kGCh = 3 * kGHead;   // conv channels of a workgroup

__device__ __forceinline__ void u4_to_f8(const vmi_u4& lo, const vmi_u4& hi, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[i] = __uint_as_float(lo[i]);
        f[4 + i] = __uint_as_float(hi[i]);
    }
}

__global__ __launch_bounds__(kGFThreads) void k_gdn_block(GdnArgs a) {
    __shared__ float s_c[kGdnMaxT][kGCh];   // conv outputs per token: q | k | v
    __shared__ float s_gb[kGdnMaxT][2];     // (g, beta) per token
    __shared__ float s_y[kGdnMaxT][kGHead];
    const int tid = threadIdx.x, lane = tid & 63, w = g_wave();
    const int h = blockIdx.x, hk = h / a.r, T = a.T;
    const int pos0 = gdn_pos0(a);

    // 1. conv operands, gate inputs and the final norm's z and weights as raw
    // values (converted after the state loads are issued; lanes without an
    // operand read zeros from an out-of-range offset), then the state rows (an
    // empty range reads zeros: nothing before position 0).  Nothing here is
    // loaded after a store: a load waits for every earlier memory operation.
    constexpr int NW = kConvTaps - 1 + kGdnMaxT;   // window: positions pos0 - 3 + i
    const bool conv_wave = w <= kGCh / 64;          // waves 0..5 conv channels, wave 6 the gates
    const int part = tid / kGHead, ch = tid % kGHead, nq = a.n_k * kGHead;
    const int c = part == 0 ? hk * kGHead + ch : part == 1 ? nq + hk * kGHead + ch : 2 * nq + h * kGHead + ch;
    const bool is_ch = tid < kGCh;
    const int src = conv_src(a, is_ch ? c : 0);
    const int gt = tid - kGCh;                      // gate token of wave 6's lanes
    const __amdgpu_buffer_rsrc_t rp = vmi_rsrc(a.proj, (uint32_t)(T * a.stride) * 4u);
    const __amdgpu_buffer_rsrc_t rr = vmi_rsrc(a.conv_ring, (uint32_t)(kConvRing * a.conv_dim) * 2u);
    const __amdgpu_buffer_rsrc_t rw = vmi_rsrc(a.conv_w, (uint32_t)(a.conv_dim * kConvTaps) * 2u);
    const __amdgpu_buffer_rsrc_t rn = vmi_rsrc(a.norm_w, kGHead * 2u);
    uint32_t rraw[kConvTaps - 1];
    float praw[kGdnMaxT];
#pragma unroll
    for (int i = 0; i < kConvTaps - 1; ++i) {
        const int p = pos0 - (kConvTaps - 1) + i;
        rraw[i] = vmi_bload_b16(rr, is_ch && p >= 0 ? (uint32_t)((p % kConvRing) * a.conv_dim + c) * 2u : VMI_OOB, 0);
    }
#pragma unroll
    for (int t = 0; t < kGdnMaxT; ++t)
        praw[t] = __uint_as_float(vmi_bload_b32(rp, is_ch && t < T ? (uint32_t)(t * a.stride + src) * 4u : VMI_OOB, 0));
    const uint2 cwraw = vmi_bload_b64(rw, is_ch ? (uint32_t)c * (kConvTaps * 2u) : VMI_OOB, 0);
    const bool is_gate = gt >= 0 && gt < T;
    const uint32_t gbase = (uint32_t)(gt * a.stride + a.n_k * a.per_g + hk * 2 * a.r + h % a.r);
    const float gb_b = __uint_as_float(vmi_bload_b32(rp, is_gate ? gbase * 4u : VMI_OOB, 0));
    const float gb_a = __uint_as_float(vmi_bload_b32(rp, is_gate ? (gbase + a.r) * 4u : VMI_OOB, 0));
    const float dtb = a.dt_bias[h], alog = a.A_log[h];
    // z of token w (wave w < T) and the norm weights of lanes l, l + 64
    const uint32_t zbase = (uint32_t)(w * a.stride + hk * a.per_g + 2 * kGHead + a.r * kGHead + (h % a.r) * kGHead + lane);
    const float z0 = __uint_as_float(vmi_bload_b32(rp, w < T ? zbase * 4u : VMI_OOB, 0));
    const float z1 = __uint_as_float(vmi_bload_b32(rp, w < T ? (zbase + 64u) * 4u : VMI_OOB, 0));
    const uint32_t nw0 = vmi_bload_b16(rn, (uint32_t)lane * 2u, 0), nw1 = vmi_bload_b16(rn, (uint32_t)(lane + 64) * 2u, 0);
    asm volatile("" ::: "memory");
    const int rowA = tid >> 4, d0 = (tid & 15) * 4;
    const size_t slot_elems = (size_t)a.n_v * kGHead * kGHead;
    const uint32_t offA = (uint32_t)(((size_t)h * kGHead + rowA) * kGHead + d0) * 4u;
    const uint32_t offB = offA + 64u * kGHead * 4u;
    const __amdgpu_buffer_rsrc_t rs =
        vmi_rsrc(a.state_ring + (size_t)(pos0 % a.n_slots) * slot_elems, pos0 > 0 ? (uint32_t)(slot_elems * 4) : 0u);
    const vmi_u4 sa0 = vmi_bload_b128_nt(rs, offA, 0), sa1 = vmi_bload_b128_nt(rs, offA + 256u, 0);
    const vmi_u4 sb0 = vmi_bload_b128_nt(rs, offB, 0), sb1 = vmi_bload_b128_nt(rs, offB + 256u, 0);

    // 2. conv and gate scalars
    const int span = a.span;
    const bool tree = a.tree_side != nullptr;
    if (conv_wave) {
        if (is_ch) {
            float ring[kConvTaps - 1];
#pragma unroll
            for (int i = 0; i < kConvTaps - 1; ++i) ring[i] = __uint_as_float(rraw[i] << 16);
            const float cw[kConvTaps] = {__uint_as_float(cwraw.x << 16), __uint_as_float(cwraw.x & 0xffff0000u),
                                         __uint_as_float(cwraw.y << 16), __uint_as_float(cwraw.y & 0xffff0000u)};
            const bool writer = part == 2 || h % a.r == 0;
            // the batch's conv inputs, rounded to bf16, into LDS (and the ring or tree_conv)
#pragma unroll
            for (int t = 0; t < kGdnMaxT; ++t) {
                if (t < T) {
                    const uint16_t b = vmi_f32_to_bf16(praw[t]);
                    s_c[t][tid] = vmi_bf16_to_f32(b);
                    if (writer) {
                        if (tree)
                            a.tree_conv[(size_t)t * a.conv_dim + c] = b;
                        else
                            a.conv_ring[(size_t)((pos0 + t) % kConvRing) * a.conv_dim + c] = b;
                    }
                }
            }
            // token t = path start + j over its window, last token first so each
            // output replaces its own input after every later token has read it
#pragma unroll
            for (int t = kGdnMaxT - 1; t >= 0; --t) {
                if (t < T) {
                    const int j = t - (t / span) * span, base = t - j;
                    float acc = 0.0f;
#pragma unroll
                    for (int tap = 0; tap < kConvTaps; ++tap) {
                        const int idx = j + tap - (kConvTaps - 1);
                        const float v = idx >= 0 ? s_c[base + idx][tid] : idx == -1 ? ring[2] : idx == -2 ? ring[1] : ring[0];
                        acc = fmaf(cw[tap], v, acc);
                    }
                    s_c[t][tid] = acc / (1.0f + expf(-acc));
                }
            }
        } else if (gt < T) {
            const float x = gb_a + dtb;
            const float sp = x > 30.0f ? x : log1pf(expf(x));
            s_gb[gt][0] = expf(-expf(alog) * sp);
            s_gb[gt][1] = 1.0f / (1.0f + expf(-gb_b));
        }
    }
    __syncthreads();

    // 3. q and k normalisation
    for (int i = w; i < 2 * T; i += kGFThreads / 64) {
        const int t = i >> 1, part = i & 1;
        float* v = &s_c[t][part * kGHead];
        const float o0 = v[lane], o1 = v[lane + 64];
        float ss = fmaf(o0, o0, o1 * o1);
        ss = vmi_wave_sum_canon(ss);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / kGHead) + 1e-6f));
        const float scale = part == 0 ? 1.0f / kGHead : 0.08838834764831845f;  // 1/128, 1/sqrt(128)
        v[lane] = o0 * inv * scale;
        v[lane + 64] = o1 * inv * scale;
    }
    __syncthreads();
    if (tree) {  // the recurrence's inputs of every token, for the commit's replay
        const int sw = a.side_stride;
        for (int i = tid; i < T * 2 * kGHead; i += kGFThreads) {
            const int t = i / (2 * kGHead), e = i - t * 2 * kGHead;
            float* row = a.tree_side + (size_t)t * sw;
            if (e < kGHead) {  // k of the key head (s_c: q | k | v)
                if (h % a.r == 0) row[hk * kGHead + e] = s_c[t][kGHead + e];
            } else {           // v of this head
                row[a.n_k * kGHead + h * kGHead + e - kGHead] = s_c[t][kGHead + e];
            }
        }
        if (tid < T) {
            float* row = a.tree_side + (size_t)tid * sw + a.n_k * kGHead + a.n_v * kGHead + 2 * h;
            row[0] = s_gb[tid][0];
            row[1] = s_gb[tid][1];
        }
    }

    // 4. delta rule
    float S0[2][8];
    u4_to_f8(sa0, sa1, S0[0]);
    u4_to_f8(sb0, sb1, S0[1]);
    for (int p = 0; p * span < T; ++p) {
        float S[2][8];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) S[j][i] = S0[j][i];
        for (int t = p * span; t < (p + 1) * span; ++t) {
            float kk[8], qq[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int d = d0 + (i & 3) + (i >> 2) * 64;
                qq[i] = s_c[t][d];
                kk[i] = s_c[t][kGHead + d];
            }
            const float g = s_gb[t][0], beta = s_gb[t][1];
            float* slot = a.state_ring + (size_t)((pos0 + t + 1) % a.n_slots) * slot_elems;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = rowA + 64 * j;
                gdn_row_update(S[j], kk, s_c[t][2 * kGHead + row], g, beta);
                float yo = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) yo = fmaf(S[j][i], qq[i], yo);
                yo = vmi_row_sum16(yo);
                if (!tree) {
                    float* dst = slot + ((size_t)h * kGHead + row) * kGHead + d0;
                    // the ring is read back at the next call at the earliest: nontemporal stores
                    const vmi_f4 lo = {S[j][0], S[j][1], S[j][2], S[j][3]}, hi = {S[j][4], S[j][5], S[j][6], S[j][7]};
                    __builtin_nontemporal_store(lo, reinterpret_cast<vmi_f4*>(dst));
                    __builtin_nontemporal_store(hi, reinterpret_cast<vmi_f4*>(dst + 64));
                }
                if ((lane & 15) == 0) s_y[t][row] = yo;
            }
        }
    }
    __syncthreads();

    // 5. gated RMSNorm
    if (w < T) {
        const int t = w;
        const float y0 = s_y[t][lane], y1 = s_y[t][lane + 64];
        float ss = fmaf(y0, y0, y1 * y1);
        ss = vmi_wave_sum_canon(ss);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / kGHead) + a.eps));
        uint16_t* o = a.o + ((size_t)t * a.n_v + h) * kGHead;
        o[lane] = vmi_f32_to_bf16(y0 * inv * __uint_as_float(nw0 << 16) * (z0 / (1.0f + expf(-z0))));
        o[lane + 64] = vmi_f32_to_bf16(y1 * inv * __uint_as_float(nw1 << 16) * (z1 / (1.0f + expf(-z1))));
    }
}

struct GdnLayout {
    size_t xn, proj, o, bytes;
};

GdnLayout gdn_layout(int T, int H, int n_k, int n_v) {
    GdnLayout L{};
    size_t off = 0;
    auto take = [&](size_t b) {
        const size_t o = off;
        off += vmi::align256(b);
        return o;
    };
    const int r = n_v / n_k;
    const int stride = n_k * (2 * kGHead + 2 * r * kGHead) + 2 * n_v;
    L.xn = take((size_t)T * H * 2);
    L.proj = take((size_t)T * stride * 4);
    L.o = take((size_t)T * n_v * kGHead * 2);
    L.bytes = off;
    return L;
}

}  // namespace

extern "C" size_t vmi_gdn_layer_workspace_bytes(int T, int hidden, int n_k_heads, int n_v_heads) {
    if (T <= 0 || hidden <= 0 || n_k_heads <= 0 || n_v_heads <= 0 || n_v_heads % n_k_heads) return 0;
    return gdn_layout(T, hidden, n_k_heads, n_v_heads).bytes;
}

namespace {

int gdn_impl(const vmi_gdn_layer_desc* desc, const uint16_t* x, int paths, int span, int pos0,
             const int32_t* pos_device, uint16_t* conv_ring, float* state_ring, int n_slots, uint16_t* tree_conv,
             float* tree_side, uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
    if (!desc) return vmi::fail(VMI_ERR_INVALID, "null desc");
    const vmi_gdn_layer_desc& D = *desc;
    const int T = paths * span;
    const bool tree = tree_side != nullptr;
    if (span <= 0 || span > kGdnMaxSpan) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d must be in [1, %d]", span, kGdnMaxSpan);
    if (paths <= 0 || T > kGdnMaxT)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "paths=%d x span=%d exceeds %d tokens", paths, span, kGdnMaxT);
    if (D.head_k_dim != kGHead || D.head_v_dim != kGHead)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "head dims %d/%d (128 only)", D.head_k_dim, D.head_v_dim);
    if (D.n_k_heads <= 0 || D.n_v_heads <= 0 || D.n_v_heads % D.n_k_heads || D.n_v_heads > 64)
        return vmi::fail(VMI_ERR_INVALID, "n_k_heads=%d n_v_heads=%d", D.n_k_heads, D.n_v_heads);
    if (D.hidden % 512 || D.hidden > 4096) return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d", D.hidden);
    const int Tp = T < 8 ? T : 8;  // tokens of one GEMV launch
    if (D.n_v_heads * kGHead * Tp > 32768 || D.hidden * Tp > 32768)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "T too large for the projection GEMV");
    if ((D.bits != 4 && D.bits != 8) || D.group != 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "bits=%d group=%d", D.bits, D.group);
    if (!pos_device && pos0 < 0) return vmi::fail(VMI_ERR_INVALID, "pos0=%d", pos0);
    if (!tree && n_slots < T + 1) return vmi::fail(VMI_ERR_INVALID, "n_slots=%d must be at least T + 1 = %d", n_slots, T + 1);
    if (n_slots < 1) return vmi::fail(VMI_ERR_INVALID, "n_slots=%d", n_slots);
    if (tree && !tree_conv) return vmi::fail(VMI_ERR_INVALID, "null tree_conv");
    if (!x || !out || !conv_ring || !state_ring || !D.input_norm || !D.conv_weight || !D.A_log || !D.dt_bias ||
        !D.norm_weight)
        return vmi::fail(VMI_ERR_INVALID, "null x/out/ring/weights");
    if (!vmi::qmat_ok(D.in_proj_qkvz) || !vmi::qmat_ok(D.in_proj_ba) || !vmi::qmat_ok(D.out_proj))
        return vmi::fail(VMI_ERR_INVALID, "projection weights must be non-null and 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(state_ring) |
         reinterpret_cast<uintptr_t>(D.input_norm)) & 15)
        return vmi::fail(VMI_ERR_INVALID, "x, out, state ring and norm weight must be 16-byte aligned");
    const GdnLayout L = gdn_layout(T, D.hidden, D.n_k_heads, D.n_v_heads);
    if (!workspace || workspace_bytes < L.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", L.bytes, workspace_bytes);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int r = D.n_v_heads / D.n_k_heads;

    GdnArgs a{};
    a.T = T; a.pos0 = pos0; a.pos_dev = pos_device; a.n_k = D.n_k_heads; a.n_v = D.n_v_heads; a.r = r;
    a.paths = paths; a.span = span; a.tree_conv = tree_conv; a.tree_side = tree_side;
    a.side_stride = vmi_gdn_tree_side_stride(D.n_k_heads, D.n_v_heads);
    a.per_g = 2 * kGHead + 2 * r * kGHead;
    a.conv_dim = 2 * D.n_k_heads * kGHead + D.n_v_heads * kGHead;
    a.stride = D.n_k_heads * a.per_g + 2 * D.n_v_heads;
    a.proj = reinterpret_cast<float*>(ws + L.proj);
    a.conv_w = D.conv_weight; a.A_log = D.A_log; a.dt_bias = D.dt_bias;
    a.conv_ring = conv_ring; a.state_ring = state_ring; a.n_slots = n_slots;
    a.norm_w = D.norm_weight; a.eps = D.norm_eps;
    a.o = reinterpret_cast<uint16_t*>(ws + L.o);
    uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);

    // input RMSNorm inside the projection when the GEMV can take it, else its own kernel
    vmi::QgemvCall q{};
    q.x = x; q.T = T; q.K = D.hidden; q.bits = D.bits;
    q.m[0] = D.in_proj_qkvz; q.m[1] = D.in_proj_ba; q.m[2] = D.in_proj_ba;
    q.rows[0] = D.n_k_heads * a.per_g; q.rows[1] = 2 * D.n_v_heads; q.rows[2] = 0;
    q.nrows = a.stride; q.out = const_cast<float*>(a.proj); q.out_stride = a.stride;
    q.norm_w = D.input_norm; q.eps = D.norm_eps;
    hipError_t e = hipSuccess;
    if (!vmi::qgemv_fuses_norm(q)) {
        e = vmi::launch_rmsnorm(x, D.input_norm, D.norm_eps, T, D.hidden, xn, s);
        if (e != hipSuccess) return vmi::hip_fail(e, "input norm launch");
        q.x = xn;
        q.norm_w = nullptr;
    }
    e = vmi::launch_qgemv(q, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "qkvz/ba projection launch");

    hipLaunchKernelGGL(k_gdn_block, dim3(D.n_v_heads), dim3(kGFThreads), 0, s, a);

    vmi::QgemvCall o{};
    o.x = a.o; o.T = T; o.K = D.n_v_heads * kGHead; o.bits = D.bits;
    o.m[0] = D.out_proj; o.m[1] = D.out_proj; o.m[2] = D.out_proj;
    o.rows[0] = D.hidden; o.rows[1] = 0; o.rows[2] = 0; o.nrows = D.hidden;
    o.out = nullptr; o.out_stride = D.hidden; o.residual = x; o.out_bf16 = out;
    e = vmi::launch_qgemv(o, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "out_proj launch");
    return VMI_OK;
}

// ------------------------------------------------------------ tree commit
// grid (heads, layers), 1024 threads.  Attention layer, kv head g < n_kv:
// the winning path's keys and values of positions pos0 .. pos0 + acc - 1 from
// tree_kv into the cache.  Gated DeltaNet layer, v-head h < n_v: its share of
// the conv channels of those positions from tree_conv into the ring, and the
// state before pos0 + acc: the state before pos0 with the winning path's
// first acc tokens applied (gdn_row_update, the thread layout of
// k_gdn_block), into ring slot (pos0 + acc) % n_slots.
struct TreeCommitArgs {
    const int32_t* rec;
    const vmi_tree_layer* layers;
    int paths, span, pos0;
    const int32_t* pos_dev;
};

__global__ __launch_bounds__(kGFThreads) void k_tree_commit(TreeCommitArgs a) {
    const vmi_tree_layer& Ly = a.layers[blockIdx.y];
    const int hh = blockIdx.x, tid = threadIdx.x;
    const int acc = a.rec[2], win = a.rec[3];
    if (acc < 1 || acc > a.span || win < 0 || win >= a.paths) return;
    const int pos0 = a.pos_dev ? max(*a.pos_dev, 0) : a.pos0;
    const int t0 = win * a.span;  // the winning path's first token
    if (Ly.kind == VMI_TREE_ATTENTION) {
        if (hh >= Ly.n_kv_heads) return;
        for (int i = tid; i < acc * 256; i += kGFThreads) {
            const int j = i >> 8, d = i & 255, pos = pos0 + j;
            if (pos >= Ly.max_len) continue;
            const uint16_t* side = Ly.tree_kv + ((size_t)(win * Ly.n_kv_heads + hh) * 2 * a.span + j) * 256;
            const size_t blk = vmi_kv_block(hh, Ly.max_len, pos);
            const int kt = pos % VMI_KV_BLOCK;
            Ly.k_cache[blk + vmi_k_elem(kt, d)] = side[d];
            Ly.v_cache[blk + vmi_v_elem(kt, d)] = side[(size_t)a.span * 256 + d];
        }
        return;
    }
    if (Ly.kind != VMI_TREE_GDN || hh >= Ly.n_v_heads) return;
    const int h = hh, n_k = Ly.n_k_heads, n_v = Ly.n_v_heads, hk = h / (n_v / n_k);
    const int conv_dim = 2 * n_k * kGHead + n_v * kGHead;
    const int c0 = h * (conv_dim / n_v), c1 = (h + 1) * (conv_dim / n_v);
    for (int i = tid; i < acc * (c1 - c0); i += kGFThreads) {
        const int j = i / (c1 - c0), c = c0 + i - j * (c1 - c0);
        Ly.conv_ring[(size_t)((pos0 + j) % kConvRing) * conv_dim + c] = Ly.tree_conv[(size_t)(t0 + j) * conv_dim + c];
    }
    const int rowA = tid >> 4, d0 = (tid & 15) * 4;
    const size_t slot_elems = (size_t)n_v * kGHead * kGHead;
    const size_t offA = ((size_t)h * kGHead + rowA) * kGHead + d0, offB = offA + 64 * kGHead;
    const float* src = Ly.state_ring + (size_t)(pos0 % Ly.n_slots) * slot_elems;
    float S[2][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        S[0][i] = pos0 > 0 ? src[offA + i] : 0.0f;
        S[0][4 + i] = pos0 > 0 ? src[offA + 64 + i] : 0.0f;
        S[1][i] = pos0 > 0 ? src[offB + i] : 0.0f;
        S[1][4 + i] = pos0 > 0 ? src[offB + 64 + i] : 0.0f;
    }
    const int sw = vmi_gdn_tree_side_stride(n_k, n_v);
    for (int j = 0; j < acc; ++j) {
        const float* row = Ly.tree_side + (size_t)(t0 + j) * sw;
        float kk[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) kk[i] = row[hk * kGHead + d0 + (i & 3) + (i >> 2) * 64];
        const float g = row[n_k * kGHead + n_v * kGHead + 2 * h], beta = row[n_k * kGHead + n_v * kGHead + 2 * h + 1];
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
            gdn_row_update(S[jj], kk, row[n_k * kGHead + h * kGHead + rowA + 64 * jj], g, beta);
    }
    float* dst = Ly.state_ring + (size_t)((pos0 + acc) % Ly.n_slots) * slot_elems;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        dst[offA + i] = S[0][i];
        dst[offA + 64 + i] = S[0][4 + i];
        dst[offB + i] = S[1][i];
        dst[offB + 64 + i] = S[1][4 + i];
    }
}

}  // namespace

extern "C" int vmi_gdn_layer(const vmi_gdn_layer_desc* desc, const uint16_t* x, int T, int pos0,
                             const int32_t* pos_device, uint16_t* conv_ring,
                             float* state_ring, int n_slots, uint16_t* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
    vmi::clear_error();
    return gdn_impl(desc, x, 1, T, pos0, pos_device, conv_ring, state_ring, n_slots, nullptr, nullptr, out,
                    workspace, workspace_bytes, stream);
}

extern "C" int vmi_gdn_tree(const vmi_gdn_layer_desc* desc, const uint16_t* x, int paths, int span, int pos0,
                            const int32_t* pos_device, const uint16_t* conv_ring, const float* state_ring,
                            int n_slots, uint16_t* tree_conv, float* tree_side, uint16_t* out, void* workspace,
                            size_t workspace_bytes, void* stream) {
    vmi::clear_error();
    if (!tree_side) return vmi::fail(VMI_ERR_INVALID, "null tree_side");
    // the rings are only read: a tree writes its conv inputs and recurrence inputs to tree_conv / tree_side
    return gdn_impl(desc, x, paths, span, pos0, pos_device, const_cast<uint16_t*>(conv_ring),
                    const_cast<float*>(state_ring), n_slots, tree_conv, tree_side, out, workspace, workspace_bytes,
                    stream);
}

extern "C" int vmi_tree_commit(const int32_t* result, const vmi_tree_layer* layers, int n_layers, int max_heads,
                               int paths, int span, int pos0, const int32_t* pos_device, void* stream) {
    vmi::clear_error();
    if (!result || !layers || n_layers <= 0 || n_layers > 65535 || max_heads <= 0 || max_heads > 64)
        return vmi::fail(VMI_ERR_INVALID, "result/layers null or n_layers=%d max_heads=%d", n_layers, max_heads);
    if (span <= 0 || span > kGdnMaxSpan || paths <= 0 || paths * span > kGdnMaxT)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "paths=%d span=%d", paths, span);
    if (!pos_device && pos0 < 0) return vmi::fail(VMI_ERR_INVALID, "pos0=%d", pos0);
    TreeCommitArgs c{result, layers, paths, span, pos0, pos_device};
    hipLaunchKernelGGL(k_tree_commit, dim3(max_heads, n_layers), dim3(kGFThreads), 0, static_cast<hipStream_t>(stream), c);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_tree_commit launch");
}
