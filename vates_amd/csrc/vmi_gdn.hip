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
//   k_rms_rows / k_qgemv (vmi_attn.hip)  input norm; qkvz and ba projections
//   k_gdn_conv    per (token, head item): conv input rows rounded to bf16 and
//                 appended to the ring, causal conv of width 4 + SiLU, q/k
//                 normalisation (rms_norm(., 1e-6) / dk and / sqrt(dk)),
//                 beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt_bias))
//   k_gdn_delta   per (v-head, 16 state rows): the delta rule over the T tokens
//                 in fp32, 16 lanes per row; state after each token to the ring
//   k_gdn_norm    gated RMSNorm per (token, v-head): y / rms * w * silu(z)
//   k_qgemv       out_proj with the residual add

#include "vmi_device.h"
#include "vmi_internal.h"

namespace {

constexpr int kGThreads = 256;
constexpr int kGHead = 128;        // head_k_dim = head_v_dim
constexpr int kConvRing = 32;      // conv ring rows
constexpr int kConvTaps = 4;
constexpr int kGdnMaxT = 8;

__device__ __forceinline__ int g_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

struct GdnArgs {
    int T, pos0, n_k, n_v, r;      // r = n_v / n_k
    const int32_t* pos_dev;        // if set: pos0 is read here (graph replays)
    int per_g, conv_dim, stride;   // proj row: [n_k groups of per_g | ba (2 n_v)]
    const float* proj;             // [T, stride] f32
    const uint16_t* conv_w;        // [conv_dim][4] bf16
    const float* A_log;            // [n_v]
    const float* dt_bias;          // [n_v]
    uint16_t* conv_ring;           // [32][conv_dim]
    float* state_ring;             // [n_slots][n_v][128][128]
    int n_slots;
    float* qk;                     // [T][2 n_k][128]: q heads then k heads, normalised and scaled
    float* v;                      // [T][n_v][128]
    float* gb;                     // [T][n_v][2]: (g, beta)
    float* y;                      // [T][n_v][128]
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

// One wave per (token, item): items 0..2 n_k - 1 are the q then k heads,
// 2 n_k .. 2 n_k + n_v - 1 the v heads, 2 n_k + n_v the gate scalars.
// Lane l owns channels l and l + 64 of the head.
__global__ __launch_bounds__(kGThreads) void k_gdn_conv(GdnArgs a) {
    const int lane = threadIdx.x & 63;
    const int items = 2 * a.n_k + a.n_v + 1;
    const int gid = blockIdx.x * (kGThreads / 64) + g_wave();
    if (gid >= a.T * items) return;
    const int t = gid / items, it = gid - t * items;
    const int pos0 = gdn_pos0(a);
    const int pos = pos0 + t;
    const float* pr = a.proj + (size_t)t * a.stride;
    if (it == items - 1) {
        for (int h = lane; h < a.n_v; h += 64) {
            const float* ba = pr + a.n_k * a.per_g + (h / a.r) * 2 * a.r;
            const float b = ba[h % a.r], av = ba[a.r + h % a.r];
            const float x = av + a.dt_bias[h];
            const float sp = x > 30.0f ? x : log1pf(expf(x));
            a.gb[((size_t)t * a.n_v + h) * 2] = expf(-expf(a.A_log[h]) * sp);
            a.gb[((size_t)t * a.n_v + h) * 2 + 1] = 1.0f / (1.0f + expf(-b));
        }
        return;
    }
    const int c0 = it * kGHead;  // first channel of the head
    float out[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int c = c0 + lane + 64 * j;
        const int src = conv_src(a, c);
        const float cur = bf16_round(pr[src]);
        a.conv_ring[(size_t)(pos % kConvRing) * a.conv_dim + c] = vmi_f32_to_bf16(cur);
        float acc = 0.0f;
#pragma unroll
        for (int tap = 0; tap < kConvTaps; ++tap) {
            const int p = pos - (kConvTaps - 1) + tap;
            float m;
            if (p == pos) m = cur;
            else if (p >= pos0) m = bf16_round(a.proj[(size_t)(p - pos0) * a.stride + src]);
            else if (p >= 0) m = vmi_bf16_to_f32(a.conv_ring[(size_t)(p % kConvRing) * a.conv_dim + c]);
            else m = 0.0f;
            acc = fmaf(vmi_bf16_to_f32(a.conv_w[(size_t)c * kConvTaps + tap]), m, acc);
        }
        out[j] = acc / (1.0f + expf(-acc));
    }
    if (it < 2 * a.n_k) {
        float ss = fmaf(out[0], out[0], out[1] * out[1]);
        ss = vmi_wave_sum_canon(ss);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / kGHead) + 1e-6f));
        const float scale = it < a.n_k ? 1.0f / kGHead : 0.08838834764831845f;  // 1/128, 1/sqrt(128)
        float* dst = a.qk + ((size_t)t * 2 * a.n_k + it) * kGHead;
        dst[lane] = out[0] * inv * scale;
        dst[lane + 64] = out[1] * inv * scale;
    } else {
        float* dst = a.v + ((size_t)t * a.n_v + (it - 2 * a.n_k)) * kGHead;
        dst[lane] = out[0];
        dst[lane + 64] = out[1];
    }
}

// 16 lanes per state row (8 dk values each), 4 rows per wave, 16 rows per
// workgroup; grid (128 / 16, n_v).  The sums over dk reduce the 16 lanes in
// a fixed butterfly, the same for every batch size, so a T-token call equals
// T one-token calls bit for bit.
__device__ __forceinline__ float sum16(float v) {
    v += __shfl_xor(v, 8);
    v += __shfl_xor(v, 4);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 1);
    return v;
}

__global__ __launch_bounds__(kGThreads) void k_gdn_delta(GdnArgs a) {
    const int lane = threadIdx.x & 63, w = g_wave();
    const int h = blockIdx.y;
    const int row = blockIdx.x * 16 + w * 4 + (lane >> 4);  // dv index
    const int d0 = (lane & 15) * 8;                          // dk slice
    const int hk = h / a.r;
    const size_t slot_elems = (size_t)a.n_v * kGHead * kGHead;
    const size_t roff = ((size_t)h * kGHead + row) * kGHead + d0;
    const int pos0 = gdn_pos0(a);
    float S[8];
    if (pos0 > 0) {
        const float* src = a.state_ring + (size_t)(pos0 % a.n_slots) * slot_elems + roff;
        const float4 u0 = *reinterpret_cast<const float4*>(src);
        const float4 u1 = *reinterpret_cast<const float4*>(src + 4);
        S[0] = u0.x; S[1] = u0.y; S[2] = u0.z; S[3] = u0.w;
        S[4] = u1.x; S[5] = u1.y; S[6] = u1.z; S[7] = u1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) S[i] = 0.0f;
    }
    for (int t = 0; t < a.T; ++t) {
        const float* kp = a.qk + ((size_t)t * 2 * a.n_k + a.n_k + hk) * kGHead + d0;
        const float* qp = a.qk + ((size_t)t * 2 * a.n_k + hk) * kGHead + d0;
        const float4 k0 = *reinterpret_cast<const float4*>(kp), k1 = *reinterpret_cast<const float4*>(kp + 4);
        const float4 q0 = *reinterpret_cast<const float4*>(qp), q1 = *reinterpret_cast<const float4*>(qp + 4);
        const float kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
        const float qq[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const float g = a.gb[((size_t)t * a.n_v + h) * 2], beta = a.gb[((size_t)t * a.n_v + h) * 2 + 1];
        const float vv = a.v[((size_t)t * a.n_v + h) * kGHead + row];
        float kv = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            S[i] *= g;
            kv = fmaf(S[i], kk[i], kv);
        }
        kv = sum16(kv);
        const float delta = (vv - kv) * beta;
        float yo = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            S[i] = fmaf(kk[i], delta, S[i]);
            yo = fmaf(S[i], qq[i], yo);
        }
        yo = sum16(yo);
        float* dst = a.state_ring + (size_t)((pos0 + t + 1) % a.n_slots) * slot_elems + roff;
        *reinterpret_cast<float4*>(dst) = make_float4(S[0], S[1], S[2], S[3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(S[4], S[5], S[6], S[7]);
        if ((lane & 15) == 0) a.y[((size_t)t * a.n_v + h) * kGHead + row] = yo;
    }
}

// One wave per (token, v-head): o = y / sqrt(mean(y^2) + eps) * w * silu(z).
__global__ __launch_bounds__(kGThreads) void k_gdn_norm(GdnArgs a) {
    const int lane = threadIdx.x & 63;
    const int gid = blockIdx.x * (kGThreads / 64) + g_wave();
    if (gid >= a.T * a.n_v) return;
    const int t = gid / a.n_v, h = gid - t * a.n_v;
    const float* y = a.y + (size_t)gid * kGHead;
    const float y0 = y[lane], y1 = y[lane + 64];
    float ss = fmaf(y0, y0, y1 * y1);
    ss = vmi_wave_sum_canon(ss);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / kGHead) + a.eps));
    const float* z = a.proj + (size_t)t * a.stride + (h / a.r) * a.per_g + 2 * kGHead + a.r * kGHead +
                     (h % a.r) * kGHead;
    const float z0 = z[lane], z1 = z[lane + 64];
    uint16_t* o = a.o + (size_t)gid * kGHead;
    o[lane] = vmi_f32_to_bf16(y0 * inv * vmi_bf16_to_f32(a.norm_w[lane]) * (z0 / (1.0f + expf(-z0))));
    o[lane + 64] = vmi_f32_to_bf16(y1 * inv * vmi_bf16_to_f32(a.norm_w[lane + 64]) * (z1 / (1.0f + expf(-z1))));
}

struct GdnLayout {
    size_t xn, proj, qk, v, gb, y, o, bytes;
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
    L.qk = take((size_t)T * 2 * n_k * kGHead * 4);
    L.v = take((size_t)T * n_v * kGHead * 4);
    L.gb = take((size_t)T * n_v * 2 * 4);
    L.y = take((size_t)T * n_v * kGHead * 4);
    L.o = take((size_t)T * n_v * kGHead * 2);
    L.bytes = off;
    return L;
}

}  // namespace

extern "C" size_t vmi_gdn_layer_workspace_bytes(int T, int hidden, int n_k_heads, int n_v_heads) {
    if (T <= 0 || hidden <= 0 || n_k_heads <= 0 || n_v_heads <= 0 || n_v_heads % n_k_heads) return 0;
    return gdn_layout(T, hidden, n_k_heads, n_v_heads).bytes;
}

extern "C" int vmi_gdn_layer(const vmi_gdn_layer_desc* desc, const uint16_t* x, int T, int pos0,
                             const int32_t* pos_device, uint16_t* conv_ring,
                             float* state_ring, int n_slots, uint16_t* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
    vmi::clear_error();
    if (!desc) return vmi::fail(VMI_ERR_INVALID, "null desc");
    const vmi_gdn_layer_desc& D = *desc;
    if (T <= 0 || T > kGdnMaxT) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d must be in [1, %d]", T, kGdnMaxT);
    if (D.head_k_dim != kGHead || D.head_v_dim != kGHead)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "head dims %d/%d (128 only)", D.head_k_dim, D.head_v_dim);
    if (D.n_k_heads <= 0 || D.n_v_heads <= 0 || D.n_v_heads % D.n_k_heads || D.n_v_heads > 64)
        return vmi::fail(VMI_ERR_INVALID, "n_k_heads=%d n_v_heads=%d", D.n_k_heads, D.n_v_heads);
    if (D.hidden % 512 || D.hidden > 4096) return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d", D.hidden);
    if (D.n_v_heads * kGHead * T > 32768 || D.hidden * T > 32768)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "T too large for the projection GEMV");
    if ((D.bits != 4 && D.bits != 8) || D.group != 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "bits=%d group=%d", D.bits, D.group);
    if (!pos_device && pos0 < 0) return vmi::fail(VMI_ERR_INVALID, "pos0=%d", pos0);
    if (n_slots < T + 1) return vmi::fail(VMI_ERR_INVALID, "n_slots=%d must be at least T + 1 = %d", n_slots, T + 1);
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
    a.per_g = 2 * kGHead + 2 * r * kGHead;
    a.conv_dim = 2 * D.n_k_heads * kGHead + D.n_v_heads * kGHead;
    a.stride = D.n_k_heads * a.per_g + 2 * D.n_v_heads;
    a.proj = reinterpret_cast<float*>(ws + L.proj);
    a.conv_w = D.conv_weight; a.A_log = D.A_log; a.dt_bias = D.dt_bias;
    a.conv_ring = conv_ring; a.state_ring = state_ring; a.n_slots = n_slots;
    a.qk = reinterpret_cast<float*>(ws + L.qk);
    a.v = reinterpret_cast<float*>(ws + L.v);
    a.gb = reinterpret_cast<float*>(ws + L.gb);
    a.y = reinterpret_cast<float*>(ws + L.y);
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

    const int items = 2 * D.n_k_heads + D.n_v_heads + 1;
    hipLaunchKernelGGL(k_gdn_conv, dim3((T * items + 3) / 4), dim3(kGThreads), 0, s, a);
    hipLaunchKernelGGL(k_gdn_delta, dim3(kGHead / 16, D.n_v_heads), dim3(kGThreads), 0, s, a);
    hipLaunchKernelGGL(k_gdn_norm, dim3((T * D.n_v_heads + 3) / 4), dim3(kGThreads), 0, s, a);

    vmi::QgemvCall o{};
    o.x = a.o; o.T = T; o.K = D.n_v_heads * kGHead; o.bits = D.bits;
    o.m[0] = D.out_proj; o.m[1] = D.out_proj; o.m[2] = D.out_proj;
    o.rows[0] = D.hidden; o.rows[1] = 0; o.rows[2] = 0; o.nrows = D.hidden;
    o.out = nullptr; o.out_stride = D.hidden; o.residual = x; o.out_bf16 = out;
    e = vmi::launch_qgemv(o, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "out_proj launch");
    return VMI_OK;
}
