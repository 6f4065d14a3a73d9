// lm_head of the verify batch and of the draft step: logits = W_lm . rmsnorm(h)
// over the full vocabulary, with the per-token argmax fused in.
//
// W is bf16 [V, H] row-major (the tied embedding of the drafter, or the
// model's head).  One workgroup per CU; each owns a contiguous range of
// 16-row vocabulary tiles and its waves take the tiles of that range in turn.
// A wave streams its tile through a ring of NBUF 4 KB LDS buffers filled by
// global_load_lds: every DMA instruction moves 4 rows x 256 contiguous bytes,
// so the weight stream is read in long contiguous runs rather than the
// 16-rows-by-64-bytes pattern an MFMA operand load would need.  Buffers are
// XOR-swizzled (16-byte unit u of row r is stored at unit u ^ r) so the
// operand reads out of LDS are free of bank conflicts.  The normalised tokens
// are staged once per workgroup in LDS as the A operand of
// v_mfma_f32_16x16x32_bf16 (A = tokens, B = W^T tile), fp32 accumulation.
//
// Argmax: every lane keeps the best (logit, row) key of its outputs; keys are
// reduced per wave, per workgroup, and the last workgroup to finish (an
// acquire/release arrival counter in the workspace, reset by that workgroup)
// reduces the per-workgroup keys.  Ties resolve to the lower vocabulary row,
// NaN ranks below every number - mx.argmax's first-maximum rule
// (mlx_streaming/mtp/generate.py:756, drafter.py:31).
//
// Top-1 probability: every lane keeps, per token, a running (maximum m,
// sum s of exp(l - m)) over its logits; the pairs merge across the 16 lanes
// of a row, the waves of the workgroup and (in the last workgroup, in a fixed
// order) the workgroups, and p = 1 / S where S = sum_j exp(l_j - max_j l):
// softmax(l)[argmax], the draft confidence of draft_adaptive
// (mlx_streaming/mtp/drafter.py:42-62, conf *= mx.softmax(lg)[d]).
//
// Semantics: generate.py:208-217 (logits = lm_head(norm(h))),
// drafter.py:20-40 (draft token = argmax of the MTP head's logits).

#include "vmi_device.h"
#include "vmi_internal.h"

namespace {

constexpr int kHeadMaxH = 2048;      // LDS holds up to this many hidden values per token
constexpr int kHeadMaxGrid = 1024;   // per-workgroup argmax keys kept in the workspace
constexpr int kHeadMaxT = 16;
constexpr int kChunk = 4096;         // bytes of one staged chunk: 16 rows x 256 B (128 hidden values)

__device__ __forceinline__ int head_wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

struct HeadArgs {
    const uint16_t* x;        // [T, H] bf16
    const uint16_t* norm_w;   // [H] bf16 or null
    float eps;
    const uint16_t* W;        // [V, H] bf16
    int T, H, V, ntiles;
    float* logits;            // [T, V] or null
    uint64_t* partial;        // [gridDim.x, kHeadMaxT] workgroup keys
    uint32_t* counter;        // arrival counter, 0 between calls
    int32_t* argmax;          // [T] or null
    float* maxval;            // [T] or null
    float* top_prob;          // [T] or null: softmax probability of the argmax
    float2* ms_partial;       // [gridDim.x, kHeadMaxT] workgroup (max, sum of exp) pairs
    int want_keys;
};

// (m, s) pairs: s = sum of exp(l - m) over a set of logits with maximum m.
// The merge is symmetric in its operands (bit for bit), so both lanes of a
// DPP or shuffle exchange hold the same result.
__device__ __forceinline__ float2 ms_merge(float2 a, float2 b) {
    const float m = fmaxf(a.x, b.x);
    return make_float2(m, a.y * __expf(a.x - m) + b.y * __expf(b.x - m));
}

template <int CTRL>
__device__ __forceinline__ float2 ms_dpp(float2 v) {
    return make_float2(vmi_dpp_f32<CTRL>(v.x), vmi_dpp_f32<CTRL>(v.y));
}

__device__ __forceinline__ float2 row_ms(float2 v) {
    v = ms_merge(v, ms_dpp<VMI_DPP_XOR1>(v));
    v = ms_merge(v, ms_dpp<VMI_DPP_XOR2>(v));
    v = ms_merge(v, ms_dpp<VMI_DPP_HALF_MIRROR>(v));
    v = ms_merge(v, ms_dpp<VMI_DPP_MIRROR>(v));
    return v;  // every lane of a 16-lane row holds its row's pair
}

__device__ __forceinline__ float2 wave_ms(float2 v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
        v = ms_merge(v, make_float2(__shfl_xor(v.x, off), __shfl_xor(v.y, off)));
    return v;
}

__device__ __forceinline__ uint64_t row_max_u64(uint64_t v) {
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_XOR1>(v));
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_XOR2>(v));
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_HALF_MIRROR>(v));
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_MIRROR>(v));
    return v;  // every lane of a 16-lane row holds its row's maximum
}

// Token t of the batch into LDS as bf16: x itself, or the RMSNorm
// bf16(x * inv_rms * w) with inv_rms from the canonical fixed-order sum (lane
// l owns the H/64 contiguous values l*H/64.., summed in order, then the
// canonical wave tree) - the order the CPU oracle restates.
__device__ void stage_token(const HeadArgs& a, int t, uint8_t* s_row) {
    const int lane = threadIdx.x & 63;
    const int cpl = a.H >> 6;        // values per lane, a multiple of 8
    const int nv = cpl >> 3;         // 16-byte vectors per lane (<= 4)
    const uint16_t* xr = a.x + (size_t)t * a.H + lane * cpl;
    uint4 xv[4];
#pragma unroll
    for (int v = 0; v < 4; ++v)
        if (v < nv) xv[v] = *reinterpret_cast<const uint4*>(xr + 8 * v);
    if (a.norm_w) {
        float ss = 0.0f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (v < nv) {
                const uint32_t q[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float lo = __uint_as_float(q[i] << 16), hi = __uint_as_float(q[i] & 0xffff0000u);
                    ss = fmaf(lo, lo, ss);
                    ss = fmaf(hi, hi, ss);
                }
            }
        }
        ss = vmi_wave_sum_canon(ss);
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / (float)a.H) + a.eps));
        const uint16_t* nw = a.norm_w + lane * cpl;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (v < nv) {
                const uint4 wv = *reinterpret_cast<const uint4*>(nw + 8 * v);
                const uint32_t q[4] = {xv[v].x, xv[v].y, xv[v].z, xv[v].w};
                const uint32_t g[4] = {wv.x, wv.y, wv.z, wv.w};
                uint32_t o[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float lo = (__uint_as_float(q[i] << 16) * inv) * __uint_as_float(g[i] << 16);
                    const float hi = (__uint_as_float(q[i] & 0xffff0000u) * inv) * __uint_as_float(g[i] & 0xffff0000u);
                    o[i] = (uint32_t)vmi_f32_to_bf16(lo) | ((uint32_t)vmi_f32_to_bf16(hi) << 16);
                }
                xv[v] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v)
        if (v < nv) *reinterpret_cast<uint4*>(s_row + 2 * (lane * cpl + 8 * v)) = xv[v];
}

// TILED: W is tile-major (vmi_head_tiles): chunk (tile, c), the 16 rows x 256
// bytes that one ring slot holds, is 4 KB of contiguous memory, so each DMA
// instruction reads 1 KB at once instead of four 256-byte runs of four rows.
template <int MAXT, int NW, int NBUF, bool TILED>
__global__ __launch_bounds__(NW * 64) void k_head(HeadArgs a) {
    constexpr int kRow = 2 * kHeadMaxH + 16;  // LDS bytes per token row (16-byte pad: conflict-free A reads)
    __shared__ __attribute__((aligned(16))) uint8_t s_x[MAXT * kRow];
    // One array per ring slot: the compiler tells LDS-DMA targets apart by
    // variable, so a read of one slot never waits for DMAs into the others.
    __shared__ __attribute__((aligned(16))) uint8_t s_w0[NW][kChunk];
    __shared__ __attribute__((aligned(16))) uint8_t s_w1[NW][kChunk];
    __shared__ __attribute__((aligned(16))) uint8_t s_w2[NBUF > 2 ? NW : 1][NBUF > 2 ? kChunk : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_w3[NBUF > 3 ? NW : 1][NBUF > 3 ? kChunk : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_w4[NBUF > 4 ? NW : 1][NBUF > 4 ? kChunk : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_w5[NBUF > 5 ? NW : 1][NBUF > 5 ? kChunk : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_w6[NBUF > 6 ? NW : 1][NBUF > 6 ? kChunk : 16];
    __shared__ __attribute__((aligned(16))) uint8_t s_w7[NBUF > 7 ? NW : 1][NBUF > 7 ? kChunk : 16];
    __shared__ uint64_t s_best[NW][MAXT];
    __shared__ float2 s_ms[NW][MAXT];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63, w = head_wave_id();
    const int T = a.T, H = a.H, V = a.V;
    for (int t = w; t < T; t += NW) stage_token(a, t, s_x + t * kRow);
    __syncthreads();

    const int G = gridDim.x, b = blockIdx.x;
    const int tb = (int)((int64_t)a.ntiles * b / G), te = (int)((int64_t)a.ntiles * (b + 1) / G);
    const int nmine = (te - tb - w + NW - 1) / NW > 0 ? (te - tb - w + NW - 1) / NW : 0;
    const int nch = H >> 7;                  // 128 hidden values per chunk
    const int total = nmine * nch;
    const size_t row_bytes = (size_t)H * 2;

    const int n = lane & 15, g = lane >> 4;  // MFMA column (vocab row in tile) / K group
    const uint8_t* wbase = reinterpret_cast<const uint8_t*>(a.W);

    // DMA of chunk q (tile j = q / nch of this wave, hidden block c = q % nch):
    // instruction i brings rows 4i..4i+3, lane l row 4i + l/16, and fetches the
    // row's 16-byte unit (l%16) ^ row so that LDS unit u of row r holds unit u ^ r.
    auto slot = [&](int u) -> uint8_t* {  // u is a constant after unrolling
        return u == 0 ? &s_w0[w][0] : u == 1 ? &s_w1[w][0] : u == 2 ? &s_w2[w][0] : u == 3 ? &s_w3[w][0]
             : u == 4 ? &s_w4[w][0] : u == 5 ? &s_w5[w][0] : u == 6 ? &s_w6[w][0] : &s_w7[w][0];
    };
    auto issue = [&](int q, uint8_t* buf) {
        const int j = q / nch, c = q - j * nch;
        const int tile = tb + w + j * NW;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 4 * i + g;
            const uint8_t* src;
            if constexpr (TILED) {  // rows past the vocabulary are the layout's zero padding
                src = wbase + ((size_t)(tile * nch + c) * 16 + r) * 256 + 16 * ((lane & 15) ^ r);
            } else {
                const int row = min(tile * 16 + r, V - 1);
                src = wbase + (size_t)row * row_bytes + 256 * c + 16 * ((lane & 15) ^ r);
            }
            vmi_lds_dma16_opaque_nt(src, buf + 1024 * i);
        }
    };

    uint64_t best[4] = {0ull, 0ull, 0ull, 0ull};
    float2 ms[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ms[r] = make_float2(-__FLT_MAX__, 0.0f);
    const bool want_prob = a.top_prob != nullptr;
    vmi_f4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const bool a_live = n < T;  // A row n is token n; rows past T stay zero

    // nch is a multiple of NBUF (H % 512 == 0 with 4 slots, H % 1024 == 0 with
    // 8), so every group of NBUF chunks lies inside one tile and the unrolled
    // body below needs no guards.
    auto consume = [&](int c, const uint8_t* buf) {
        const uint8_t* xrow = s_x + n * kRow + 256 * c;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const vmi_u4 bv = *reinterpret_cast<const vmi_u4*>(buf + 256 * n + 16 * ((4 * m + g) ^ n));
            vmi_u4 av = {0u, 0u, 0u, 0u};
            if (a_live) av = *reinterpret_cast<const vmi_u4*>(xrow + 64 * m + 16 * g);
            acc = vmi_mfma_bf16(av, bv, acc);
        }
    };

    // A wave without tiles (small vocabularies) issues nothing: every DMA
    // below addresses a chunk in [0, total).
    if (total > 0) {
#pragma unroll
    for (int u = 0; u < NBUF - 1; ++u) issue(min(u, total - 1), slot(u));
#pragma unroll 1
    for (int j = 0; j < nmine; ++j) {
#pragma unroll 1
        for (int c0 = 0; c0 < nch; c0 += NBUF) {
#pragma unroll
            for (int u = 0; u < NBUF; ++u) {
                const int q = j * nch + c0 + u;
                // Refill the slot the previous step read (its LDS reads retire
                // first).  Past the end the last chunk is fetched again into
                // slots that are never read.
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
                issue(min(q + NBUF - 1, total - 1), slot((u + NBUF - 1) % NBUF));
                wait_vmcnt<4 * (NBUF - 1)>();
                consume(c0 + u, slot(u));
            }
        }
        // D[token 4g + r][vocab row n] sits in acc[r].
        const int row = (tb + w + j * NW) * 16 + n;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 4 * g + r;
            if (t < T && row < V) {
                if (a.logits) a.logits[(size_t)t * V + row] = acc[r];
                best[r] = vmi_u64_max(best[r], vmi_rank_key(acc[r], row));
                if (want_prob) ms[r] = ms_merge(ms[r], make_float2(acc[r], 1.0f));
            }
        }
        acc = vmi_f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    }
    wait_vmcnt<0>();
    if (!a.want_keys) return;

#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const uint64_t k = row_max_u64(best[r]);
        const int t = 4 * g + r;
        if (n == 0 && t < MAXT) s_best[w][t] = k;
        if (want_prob) {
            const float2 v = row_ms(ms[r]);
            if (n == 0 && t < MAXT) s_ms[w][t] = v;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int t = 0; t < T; ++t) {
            uint64_t k = 0ull;
            for (int v = 0; v < NW; ++v) k = vmi_u64_max(k, s_best[v][t]);
            __hip_atomic_store(&a.partial[(size_t)b * kHeadMaxT + t], k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (want_prob) {
                float2 m = s_ms[0][t];
                for (int v = 1; v < NW; ++v) m = ms_merge(m, s_ms[v][t]);
                float* dst = reinterpret_cast<float*>(&a.ms_partial[(size_t)b * kHeadMaxT + t]);
                __hip_atomic_store(dst, m.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(dst + 1, m.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        const uint32_t prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (uint32_t)(G - 1));
    }
    __syncthreads();
    if (!s_last) return;
    for (int t = w; t < T; t += NW) {
        uint64_t k = 0ull;
        for (int i = lane; i < G; i += 64)
            k = vmi_u64_max(k, __hip_atomic_load(&a.partial[(size_t)i * kHeadMaxT + t], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT));
        k = vmi_wave_max_u64(k);
        if (lane == 0) {
            if (a.argmax) a.argmax[t] = (int32_t)(0xffffffffu - (uint32_t)k);
            if (a.maxval) a.maxval[t] = vmi_order_key_value((uint32_t)(k >> 32));
        }
        if (want_prob) {
            // lane l merges workgroups l, l + 64, ... in order, then a fixed tree
            float2 m = make_float2(-__FLT_MAX__, 0.0f);
            for (int i = lane; i < G; i += 64) {
                const float* src = reinterpret_cast<const float*>(&a.ms_partial[(size_t)i * kHeadMaxT + t]);
                m = ms_merge(m, make_float2(__hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                                            __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
            }
            m = wave_ms(m);
            if (lane == 0) a.top_prob[t] = 1.0f / m.y;
        }
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Top-k (k <= 16) of each row of f32 logits [rows, V]: one workgroup per row.
// Every lane keeps its k best rank keys (value desc, lower index first, NaN
// last) over a strided pass; k rounds of a workgroup-wide maximum (wave max,
// then the 4 waves through LDS) pop the winners in order.
struct TopkArgs {
    const float* logits;
    int V, k;
    int32_t* ids;    // [rows, k]
    float* vals;     // [rows, k] or null
};

__global__ __launch_bounds__(256) void k_topk_rows(TopkArgs a) {
    __shared__ uint64_t s_w[4];
    const int lane = threadIdx.x & 63, w = head_wave_id(), r = blockIdx.x;
    const float* row = a.logits + (size_t)r * a.V;
    uint64_t best[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) best[i] = 0ull;
    for (int j = threadIdx.x; j < a.V; j += 256) {
        uint64_t key = vmi_rank_key(row[j], j);
        if (row[j] != row[j]) key = (uint64_t)(0xffffffffu - (uint32_t)j);  // NaN: below every number
        // insert into the sorted (descending) list of length k
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            if (i < a.k && key > best[i]) {
                const uint64_t t = best[i];
                best[i] = key;
                key = t;
            }
        }
    }
    for (int j = 0; j < a.k; ++j) {
        const uint64_t m = vmi_wave_max_u64(best[0]);
        if (lane == 0) s_w[w] = m;
        __syncthreads();
        const uint64_t M = vmi_u64_max(vmi_u64_max(s_w[0], s_w[1]), vmi_u64_max(s_w[2], s_w[3]));
        __syncthreads();
        if (best[0] == M) {
#pragma unroll
            for (int i = 0; i < 15; ++i) best[i] = best[i + 1];
            best[15] = 0ull;
        }
        if (threadIdx.x == 0) {
            const int idx = (int)(0xffffffffu - (uint32_t)M);
            a.ids[r * a.k + j] = idx;
            if (a.vals) a.vals[r * a.k + j] = row[idx];
        }
    }
}

}  // namespace

namespace {
constexpr size_t kKeysBytes = (size_t)kHeadMaxGrid * kHeadMaxT * sizeof(uint64_t);
constexpr size_t kMsBytes = (size_t)kHeadMaxGrid * kHeadMaxT * sizeof(float2);
// Tile-major copy of a row-major bf16 [V, H] head: 16-byte unit u of row r
// of chunk (tile, c) - vocabulary row 16 tile + r, hidden values
// 128 c + 8 u .. + 7 - goes to unit ((tile (H / 128) + c) 16 + r) 16 + u;
// rows past V are zeros.  One thread per destination unit.
__global__ __launch_bounds__(256) void k_head_tiles(const uint4* __restrict__ W, int V, int H, size_t units,
                                                    uint4* __restrict__ out) {
    const size_t d = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (d >= units) return;
    const int nch = H >> 7;
    const int u = (int)(d & 15), r = (int)((d >> 4) & 15);
    const size_t tc = d >> 8;
    const int c = (int)(tc % (size_t)nch);
    const size_t row = (tc / (size_t)nch) * 16 + r;
    out[d] = row < (size_t)V ? W[row * (size_t)(H >> 3) + (size_t)c * 16 + u] : make_uint4(0u, 0u, 0u, 0u);
}

}  // namespace

extern "C" size_t vmi_head_tiles_bytes(int vocab, int hidden) {
    if (vocab <= 0 || hidden <= 0 || hidden % 128) return 0;
    return (size_t)((vocab + 15) / 16) * 16 * (size_t)hidden * 2;
}

extern "C" int vmi_head_tiles(const uint16_t* weight, int vocab, int hidden, uint16_t* out, void* stream) {
    vmi::clear_error();
    if (vocab <= 0 || hidden <= 0 || hidden % 512 || hidden > kHeadMaxH)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "vocab=%d hidden=%d (hidden a multiple of 512 up to %d)", vocab, hidden,
                         kHeadMaxH);
    if (!weight || !out) return vmi::fail(VMI_ERR_INVALID, "null weight/out");
    if ((reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out)) & 15)
        return vmi::fail(VMI_ERR_INVALID, "weight and out must be 16-byte aligned");
    if (weight == out) return vmi::fail(VMI_ERR_INVALID, "weight and out must not alias");
    const size_t units = vmi_head_tiles_bytes(vocab, hidden) / 16;
    hipLaunchKernelGGL(k_head_tiles, dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), reinterpret_cast<const uint4*>(weight), vocab, hidden, units,
                       reinterpret_cast<uint4*>(out));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_head_tiles launch");
    return VMI_OK;
}

extern "C" size_t vmi_lm_head_workspace_bytes(int T, int vocab) {
    if (T <= 0 || vocab <= 0) return 0;
    return vmi::align256(kKeysBytes) + vmi::align256(kMsBytes) + 256;
}

static int lm_head_call(const uint16_t* x, int T, int hidden, const uint16_t* norm_weight, float norm_eps,
                        const uint16_t* weight, int vocab, float* logits, int32_t* argmax, float* max_logit,
                        float* top_prob, void* workspace, size_t workspace_bytes, void* stream, bool tiled) {
    vmi::clear_error();
    if (T <= 0 || T > kHeadMaxT) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d must be in [1, %d]", T, kHeadMaxT);
    if (hidden <= 0 || hidden % 512 || hidden > kHeadMaxH)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d must be a multiple of 512 up to %d", hidden, kHeadMaxH);
    if (vocab <= 0) return vmi::fail(VMI_ERR_INVALID, "vocab=%d", vocab);
    if ((size_t)vocab * (size_t)hidden * 2 > ((size_t)1 << 40)) return vmi::fail(VMI_ERR_UNSUPPORTED, "head too large");
    if (!x || !weight) return vmi::fail(VMI_ERR_INVALID, "null x/weight");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) |
         reinterpret_cast<uintptr_t>(norm_weight)) & 15)
        return vmi::fail(VMI_ERR_INVALID, "x, weight and norm_weight must be 16-byte aligned");
    const bool want_keys = argmax || max_logit || top_prob;
    if (!logits && !want_keys)
        return vmi::fail(VMI_ERR_INVALID, "nothing to compute (logits, argmax, max and top_prob all null)");
    const size_t need = vmi_lm_head_workspace_bytes(T, vocab);
    if (want_keys && (!workspace || workspace_bytes < need))
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", need, workspace_bytes);

    HeadArgs a{};
    a.x = x; a.norm_w = norm_weight; a.eps = norm_eps; a.W = weight;
    a.T = T; a.H = hidden; a.V = vocab; a.ntiles = (vocab + 15) / 16;
    a.logits = logits; a.argmax = argmax; a.maxval = max_logit; a.top_prob = top_prob;
    a.want_keys = want_keys ? 1 : 0;
    if (want_keys) {
        uint8_t* ws = static_cast<uint8_t*>(workspace);
        a.partial = reinterpret_cast<uint64_t*>(ws);
        a.ms_partial = reinterpret_cast<float2*>(ws + vmi::align256(kKeysBytes));
        a.counter = reinterpret_cast<uint32_t*>(ws + vmi::align256(kKeysBytes) + vmi::align256(kMsBytes));
    }
    int G = vmi::device_cus();
    if (G > kHeadMaxGrid) G = kHeadMaxGrid;
    if (G > a.ntiles) G = a.ntiles;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (tiled) {
        if (T <= 4 && hidden % 1024 == 0)
            hipLaunchKernelGGL((k_head<4, 4, 8, true>), dim3(G), dim3(4 * 64), 0, s, a);
        else if (T <= 4)
            hipLaunchKernelGGL((k_head<4, 8, 4, true>), dim3(G), dim3(8 * 64), 0, s, a);
        else
            hipLaunchKernelGGL((k_head<16, 8, 2, true>), dim3(G), dim3(8 * 64), 0, s, a);
    } else {
        if (T <= 4 && hidden % 1024 == 0)
            hipLaunchKernelGGL((k_head<4, 4, 8, false>), dim3(G), dim3(4 * 64), 0, s, a);
        else if (T <= 4)
            hipLaunchKernelGGL((k_head<4, 8, 4, false>), dim3(G), dim3(8 * 64), 0, s, a);
        else
            hipLaunchKernelGGL((k_head<16, 8, 2, false>), dim3(G), dim3(8 * 64), 0, s, a);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return vmi::hip_fail(e, "k_head launch");
    return VMI_OK;
}

extern "C" int vmi_lm_head(const uint16_t* x, int T, int hidden, const uint16_t* norm_weight, float norm_eps,
                           const uint16_t* weight, int vocab, float* logits, int32_t* argmax, float* max_logit,
                           float* top_prob, void* workspace, size_t workspace_bytes, void* stream) {
    return lm_head_call(x, T, hidden, norm_weight, norm_eps, weight, vocab, logits, argmax, max_logit, top_prob,
                        workspace, workspace_bytes, stream, false);
}

extern "C" int vmi_lm_head_tiled(const uint16_t* x, int T, int hidden, const uint16_t* norm_weight, float norm_eps,
                                 const uint16_t* tiles, int vocab, float* logits, int32_t* argmax, float* max_logit,
                                 float* top_prob, void* workspace, size_t workspace_bytes, void* stream) {
    return lm_head_call(x, T, hidden, norm_weight, norm_eps, tiles, vocab, logits, argmax, max_logit, top_prob,
                        workspace, workspace_bytes, stream, true);
}

extern "C" int vmi_topk_rows(const float* logits, int rows, int vocab, int k, int32_t* ids, float* vals, void* stream) {
    vmi::clear_error();
    if (rows <= 0 || vocab <= 0 || k <= 0 || k > 16 || k > vocab)
        return vmi::fail(VMI_ERR_INVALID, "rows=%d vocab=%d k=%d (k <= 16)", rows, vocab, k);
    if (!logits || !ids) return vmi::fail(VMI_ERR_INVALID, "null logits/ids");
    TopkArgs a{logits, vocab, k, ids, vals};
    hipLaunchKernelGGL(k_topk_rows, dim3(rows), dim3(256), 0, static_cast<hipStream_t>(stream), a);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_topk_rows launch");
}

