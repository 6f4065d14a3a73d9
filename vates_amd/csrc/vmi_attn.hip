// Full-attention decoder block of the verify batch and of the MTP draft step
// (Qwen3-Next gated attention: GQA, per-head q/k RMSNorm, partial rotary
// embedding, sigmoid output gate), and the quantised GEMV it is built on.
//
// The reference runs this block through mlx-lm's Qwen3NextAttention inside the
// MTP layer (mlx_streaming/mtp/qwen3_next_mtp.py:34-57, layer(x) at :53) and in
// the main model's full-attention layers (generate.py:101-220).  The same
// architecture is published in Hugging Face transformers' modeling_qwen3_next
// (Qwen3NextAttention: q_proj emits [q | gate] per head, q_norm/k_norm over
// head_dim, rotary on the first rotary_dim dims with rotate_half pairs
// (i, i + rotary_dim/2), softmax(q k^T / sqrt(head_dim)) v, times
// sigmoid(gate), o_proj).
//
// Kernels:
//   k_rms_rows     bf16(x * inv_rms * w) per token (canonical fixed order)
//   k_qgemv        y[t][n] = sum_k x[t][k] W[n][k], 4/8-bit affine W, T <= 8:
//                  one wave per output row, 16 bytes of packed weights per
//                  lane per step, tokens staged in LDS, fp32 accumulation
//   k_attn_chunk   per (kv head, chunk of 256, 288 or 320 keys: 8 + NX
//                  blocks of 32, NX set by the cache capacity so that one
//                  workgroup per CU covers the cache), 8 waves: while the
//                  chunk's keys and values stream in, the workgroup forms the
//                  head group's queries (q RMSNorm, rotary, bf16) and, in the
//                  chunk holding a batch position, that position's key and
//                  value (k RMSNorm, rotary), appended to the cache and put
//                  into the loaded operands; wave w scores the 32-key block w
//                  (waves x < NX also block 8 + x, staged in LDS) against the
//                  query rows (S^T = K Q^T), the chunk max and the bf16
//                  probabilities go through LDS, then wave w forms P V for
//                  dims 32w..32w+31 over all the chunk's keys; writes (max, sum, O)
//   k_attn_merge   per (token, head, quarter of the dims): merges the chunks
//                  in a fixed order, times sigmoid(gate), bf16 input of o_proj
//
// KV cache layout: per kv head, blocks of 32 positions x 256 dims (8192 bf16,
// 16 KB), each stored in the operand order of the MFMA that reads it, so every
// load of the attention kernel is a contiguous 1 KB per wave:
//   keys   element ((a*8 + kk)*64 + q4*16 + nl)*8 + e holds position
//          kt = 8*(nl>>2) + 4*a + (nl&3) of the block, dim 32*kk + 8*q4 + e
//          (the A operand of S^T = K Q^T: result row 4*q4 + r of tile a is
//          then key 8*q4 + 4*a + r, so a lane's 8 scores are 8 consecutive
//          keys, already the A operand of P V);
//   values element ((dt*64 + q4*16 + nl)*8 + e) holds position 8*q4 + e,
//          dim 16*dt + nl (the B operand of P V).

#include <type_traits>

#include "vmi_device.h"
#include "vmi_internal.h"

VMI_TL_DECL

namespace {

constexpr int kAThreads = 256;
constexpr int kQgMaxT = 8;       // tokens of one GEMV launch (and of one attention path)
constexpr int kQgMaxBatch = 16;  // tokens of a GEMV call (launched in pieces of kQgMaxT)
constexpr int kHeadDim = 256;

// The batch's first position: the argument, or read on the device (graph
// replays), clamped so that pos0 + T <= max_len.
__device__ __forceinline__ int batch_pos0(int pos0, const int32_t* pos_dev, int T, int max_len) {
    const int p = pos_dev ? *pos_dev : pos0;
    return min(max(p, 0), max_len - T);
}

__device__ __forceinline__ int at_wave() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ void bf16x8f(const uint4& q, float (&v)[8]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

// ---------------------------------------------------------------- RMSNorm
struct RmsArgs {
    const uint16_t* x;   // [T, H], or a table [rows, H] gathered through ids
    const uint16_t* w;   // [H]
    float eps;
    int T, H;
    uint16_t* out;       // [T, H]
    const int32_t* ids;  // [T] row of x per token, or null
    int rows;            // table rows (ids range)
    uint32_t* status;    // optional: VMI_STATUS_BAD_SLOT for an id out of range
    int out_stride;      // elements between output rows
};

// One wave per token; lane l owns H/64 contiguous values (H % 512 == 0).
__global__ __launch_bounds__(kAThreads) void k_rms_rows(RmsArgs a) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (kAThreads / 64) + at_wave();
    if (t >= a.T) return;
    const int cpl = a.H / 64, nv = cpl / 8;
    int row = t;
    if (a.ids) {
        row = a.ids[t];
        if (row < 0 || row >= a.rows) {
            if (lane == 0 && a.status) atomicOr(a.status, VMI_STATUS_BAD_SLOT);
            row = 0;
        }
    }
    const uint16_t* xr = a.x + (size_t)row * a.H + lane * cpl;
    float ss = 0.0f;
    for (int v = 0; v < nv; ++v) {
        float f[8];
        bf16x8f(*reinterpret_cast<const uint4*>(xr + 8 * v), f);
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
    }
    uint16_t* orow = a.out + (size_t)t * a.out_stride + lane * cpl;
    if (!a.w) {  // plain gather
        for (int v = 0; v < nv; ++v)
            *reinterpret_cast<uint4*>(orow + 8 * v) = *reinterpret_cast<const uint4*>(xr + 8 * v);
        return;
    }
    ss = vmi_wave_sum_canon(ss);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / (float)a.H) + a.eps));
    for (int v = 0; v < nv; ++v) {
        float f[8], g[8];
        bf16x8f(*reinterpret_cast<const uint4*>(xr + 8 * v), f);
        bf16x8f(*reinterpret_cast<const uint4*>(a.w + lane * cpl + 8 * v), g);
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o[i] = vmi_pack_bf16x2((f[2 * i] * inv) * g[2 * i], (f[2 * i + 1] * inv) * g[2 * i + 1]);
        *reinterpret_cast<uint4*>(orow + 8 * v) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// ------------------------------------------------------------------ GEMV
// Up to three weight matrices stacked along the output rows (q, k, v).
using QgArgs = vmi::QgemvCall;

// One wave per output row, 4 rows per workgroup.  Lane l takes 32-column
// blocks l, l + 64, ...; per block sum_c x_c q_c and sum_c x_c meet the
// block's group scale and bias once.
__global__ __launch_bounds__(kAThreads) void k_qgemv(QgArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t s_x[];  // [T][K]
    const int lane = threadIdx.x & 63, w = at_wave();
    const int T = a.T, K = a.K;
    for (int i = threadIdx.x * 8; i < T * K; i += kAThreads * 8)
        *reinterpret_cast<uint4*>(&s_x[i]) = *reinterpret_cast<const uint4*>(&a.x[i]);
    __syncthreads();
    const int n = blockIdx.x * (kAThreads / 64) + w;
    if (n >= a.nrows) return;
    int mi = 0, r = n;
    while (mi < 2 && r >= a.rows[mi]) r -= a.rows[mi++];
    const vmi_qmat M = a.m[mi];
    const int G = K / 64;
    const int wpr = K * a.bits / 32;
    float acc[kQgMaxT];
#pragma unroll
    for (int t = 0; t < kQgMaxT; ++t) acc[t] = 0.0f;
    for (int blk = lane; blk < K / 32; blk += 64) {
        const int c0 = 32 * blk;
        float wq[32];
        if (a.bits == 4) {
            const uint4 p = *reinterpret_cast<const uint4*>(M.w + (size_t)r * wpr + c0 / 8);
            const uint32_t ww[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
            for (int i = 0; i < 32; ++i) wq[i] = (float)((ww[i >> 3] >> (4 * (i & 7))) & 0xFu);
        } else {
            const uint4 p0 = *reinterpret_cast<const uint4*>(M.w + (size_t)r * wpr + c0 / 4);
            const uint4 p1 = *reinterpret_cast<const uint4*>(M.w + (size_t)r * wpr + c0 / 4 + 4);
            const uint32_t ww[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int i = 0; i < 32; ++i) wq[i] = (float)((ww[i >> 2] >> (8 * (i & 3))) & 0xFFu);
        }
        const float sc = vmi_bf16_to_f32(M.s[(size_t)r * G + c0 / 64]);
        const float bi = vmi_bf16_to_f32(M.b[(size_t)r * G + c0 / 64]);
#pragma unroll
        for (int t = 0; t < kQgMaxT; ++t) {
            if (t < T) {
                float xq = 0.0f, xs = 0.0f;
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    float xf[8];
                    bf16x8f(*reinterpret_cast<const uint4*>(&s_x[t * K + c0 + 8 * v]), xf);
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        xq = fmaf(xf[i], wq[8 * v + i], xq);
                        xs += xf[i];
                    }
                }
                acc[t] = fmaf(xq, sc, fmaf(xs, bi, acc[t]));
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kQgMaxT; ++t) {
        if (t < T) {
            const float y = vmi_wave_sum_canon(acc[t]);
            if (lane == 0) {
                if (a.out) a.out[(size_t)t * a.out_stride + n] = y;
                if (a.out_bf16) {
                    const float rr = a.residual ? vmi_bf16_to_f32(a.residual[(size_t)t * a.out_stride + n]) : 0.0f;
                    a.out_bf16[(size_t)t * a.out_stride + n] = vmi_f32_to_bf16(y + rr);
                }
            }
        }
    }
}

// ------------------------------------------------------- q/k norm, rotary
// ------------------------------------------------------------ KV cache
constexpr int kKvBlock = 32;                      // positions per cache block
constexpr int kKvBlockElems = kKvBlock * kHeadDim;

static_assert(kKvBlock == VMI_KV_BLOCK, "cache block");
__device__ __forceinline__ size_t kv_block(int g, int max_len, int pos) { return vmi_kv_block(g, max_len, pos); }
__device__ __forceinline__ int k_elem(int kt, int d) { return vmi_k_elem(kt, d); }
__device__ __forceinline__ int v_elem(int kt, int d) { return vmi_v_elem(kt, d); }

// -------------------------------------------------------------- attention
struct AttnArgs {
    const float* qkv;         // [T, stride]: q|gate per head (n_heads * 2 * 256), then k (n_kv * 256), then v
    int stride;
    const uint16_t* q_norm;   // [256]
    const uint16_t* k_norm;   // [256]
    int rope_dim;
    float eps;
    double rope_base;         // theta^(-2/rope_dim), in double
    uint16_t* k_cache;        // blocks of 32 positions, see the layout above
    uint16_t* v_cache;
    int T, n_heads, n_kv, pos0, max_len;
    int paths, span;          // T = paths * span: path p's tokens p*span .. at positions pos0 ..
    int chunks;               // chunks of the cache capacity the grid covers
    uint16_t* tree_kv;        // or null: [paths][n_kv][2][span][256] new keys/values instead of the cache
    const int32_t* pos_dev;   // if set: pos0 is read here
    uint32_t* status;         // workspace status word (VMI_STATUS_BAD_POS)
    int nstride;              // chunk capacity of the partial buffers
    uint16_t* part_o;         // [n_kv, nstride, RP, 256] bf16 (unnormalised P V of each chunk)
    float* part_ml;           // [n_kv, nstride, RP, 2]
    uint16_t* o;              // [T, n_heads * 256] bf16 gated attention output
    int chunk_keys;           // keys per chunk: 32 (8 + extra blocks)
};

constexpr int kChunkWaves = 8;                         // one cache block per wave
constexpr int kChunkThreads = 64 * kChunkWaves;
constexpr int kChunkKeys = kChunkWaves * kKvBlock;     // 256: the shortest chunk
constexpr int kMaxExtraBlocks = 2;                     // blocks per chunk beyond one per wave

__device__ __forceinline__ vmi_u4 keep_first(vmi_u4 v, int n) {  // zero bf16 elements e >= n
#pragma unroll
    for (int i = 0; i < 4; ++i)
        v[i] &= (2 * i < n ? 0x0000ffffu : 0u) | (2 * i + 1 < n ? 0xffff0000u : 0u);
    return v;
}

// NR head rows of one wave (dims lane + 64 j of row i in v[i]) in place:
// RMSNorm (x^2 of the lane's four dims in order, then the canonical wave
// sum), times the norm weight, rounded to bf16 (the model dtype), then the
// rotary pairs (d, d + rd/2) in fp32 with (cos, sin) of pos * theta^(-2i/rd)
// from cs[i], rounded to bf16.  The rows go through together and nothing
// branches on the lane, so their reductions and LDS reads overlap.  The
// rotary partner of dim d: for rd = 64 the lane 32 apart, for rd = 128 and
// 256 another register of the same lane; other widths go through srow, the
// wave's own LDS row, one row at a time.
template <int NR>
__device__ __forceinline__ void norm_rope_rows(float (&v)[NR][4], const float (&nw)[4], float eps,
                                               const float2* const (&cs)[NR], int rd, float* srow,
                                               uint16_t (&o)[NR][4]) {
    const int lane = threadIdx.x & 63;
    float ss[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        ss[i] = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) ss[i] = fmaf(v[i][j], v[i][j], ss[i]);
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) ss[i] = vmi_wave_sum_canon(ss[i]);
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const float inv = __fdiv_rn(1.0f, __fsqrt_rn(ss[i] * (1.0f / (float)kHeadDim) + eps));
        const uint32_t u01 = vmi_pack_bf16x2((v[i][0] * inv) * nw[0], (v[i][1] * inv) * nw[1]);
        const uint32_t u23 = vmi_pack_bf16x2((v[i][2] * inv) * nw[2], (v[i][3] * inv) * nw[3]);
        v[i][0] = __uint_as_float(u01 << 16);
        v[i][1] = __uint_as_float(u01 & 0xffff0000u);
        v[i][2] = __uint_as_float(u23 << 16);
        v[i][3] = __uint_as_float(u23 & 0xffff0000u);
    }
    const int half = rd / 2;
    auto store = [&](int i, const float (&r)[4]) {
        const uint32_t a = vmi_pack_bf16x2(r[0], r[1]), b = vmi_pack_bf16x2(r[2], r[3]);
        o[i][0] = (uint16_t)a;
        o[i][1] = (uint16_t)(a >> 16);
        o[i][2] = (uint16_t)b;
        o[i][3] = (uint16_t)(b >> 16);
    };
    if (rd == 64 || rd == 128 || rd == 256) {
        // register j of every lane is rotated or not as a whole (rd is a
        // multiple of 64): the table reads need no lane mask
        float2 c[NR][4];
#pragma unroll
        for (int i = 0; i < NR; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = lane + 64 * j;
                c[i][j] = 64 * j < rd ? cs[i][d < half ? d : d - half] : make_float2(1.0f, 0.0f);
            }
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            float pr[4];
            if (rd == 64) {
                pr[0] = __shfl_xor(v[i][0], 32, 64);
                pr[1] = pr[2] = pr[3] = 0.0f;
            } else if (rd == 128) {
                pr[0] = v[i][1];
                pr[1] = v[i][0];
                pr[2] = pr[3] = 0.0f;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) pr[j] = v[i][j ^ 2];
            }
            float r[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int d = lane + 64 * j;
                const float partner = d < half ? -pr[j] : pr[j];
                r[j] = 64 * j < rd ? v[i][j] * c[i][j].x + partner * c[i][j].y : v[i][j];
            }
            store(i, r);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < NR; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) srow[lane + 64 * j] = v[i][j];
        __builtin_amdgcn_wave_barrier();  // srow is this wave's own row: LDS order within a wave suffices
        float r[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            r[j] = v[i][j];
            if (d < rd) {
                const float2 c = cs[i][d < half ? d : d - half];
                const float partner = d < half ? -srow[d + half] : srow[d - half];
                r[j] = v[i][j] * c.x + partner * c.y;
            }
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read its partner before srow is rewritten
        store(i, r);
    }
}

// Rows of a head group: row = t * G + hl (G = n_heads / n_kv query heads per
// kv head), RP = 16 MS >= T * G.  A chunk is NB = 8 + NX blocks of 32 keys:
// wave w scores block w from registers, and waves x < NX also score block
// 8 + x, whose keys every wave helps stage in LDS (2 KB each).  Loads in issue
// order: the projections of the wave's query rows (rows w, w + 8, ...), in the
// chunk holding batch positions the key and value projections of one of them
// per wave, then the keys of the wave's block (16 x 1 KB), its share of the
// extra blocks' keys, and values of all NB blocks for the wave's 32 dims
// (2 NB x 1 KB); the queries and new keys are formed while the cache streams.  Positions >= pos0 + T are not read past their block; inside
// the last block they are masked (scores -inf, values zeroed), so stale cache
// contents never reach the result.  The batch's own positions are read from
// the cache too, before this workgroup writes them: their operands are then
// replaced by the new keys and values.
template <int MS, int NX>
__global__ __launch_bounds__(kChunkThreads) void k_attn_chunk(AttnArgs a) {
    constexpr int RP = 16 * MS;
    constexpr int NB = kChunkWaves + NX;  // blocks per chunk
    constexpr int CK = NB * kKvBlock;     // keys per chunk
    static_assert(NX >= 0 && NX <= kMaxExtraBlocks, "extra blocks");
    __shared__ __attribute__((aligned(16))) uint16_t s_q[RP][kHeadDim + 8];
    __shared__ vmi_u4 s_pa[MS][NB][64];
    __shared__ vmi_u4 s_kx[NX > 0 ? NX : 1][16][64];  // keys of block 8 + x, operand order
    __shared__ float s_wm[kChunkWaves][RP], s_wl[kChunkWaves][RP];
    // chunks in reverse launch order: the last (partly filled) chunk and those
    // past the cache take the first CUs and free them early
    __shared__ float s_row[kChunkWaves][kHeadDim];                  // a wave's normalised row
    __shared__ float2 s_cs[kQgMaxT][kHeadDim / 2];                  // (cos, sin) per (token, frequency)
    __shared__ __attribute__((aligned(16))) uint16_t s_new[2][kQgMaxT][kHeadDim];  // new keys, values (bf16)
    // one path: chunk gridDim.x - 1 - blockIdx.x.  Several (a tree): groups of
    // 8 chunks x paths, a chunk's paths 8 apart in launch order (the same XCD,
    // hence one L2 fetch of its cache blocks for all paths).
    const int P = a.paths, T = a.span;                // T: this workgroup's tokens (one path)
    int c, p = 0;
    if (P == 1) {
        c = gridDim.x - 1 - blockIdx.x;
    } else {
        const int grp = blockIdx.x / (8 * P), rem = blockIdx.x - grp * 8 * P;
        p = rem >> 3;
        c = a.chunks - 1 - (grp * 8 + (rem & 7));
        if (c < 0) return;
    }
    const int g = blockIdx.y, tid = threadIdx.x;
    VMI_STAMP(4 + g, 0);
    const int lane = tid & 63, w = at_wave(), nl = lane & 15, q4 = lane >> 4;
    const int G = a.n_heads / a.n_kv, R = T * G;
    const int tok0 = p * T;                            // the path's first row of qkv
    const int pos0 = batch_pos0(a.pos0, a.pos_dev, T, a.max_len);
    if (a.pos_dev && blockIdx.x == 0 && g == 0 && tid == 0 && *a.pos_dev != pos0)
        atomicOr(a.status, VMI_STATUS_BAD_POS);    // clamped: the caller's position overran the cache
    const int L = pos0 + T;                            // positions present
    if (c * CK >= L) return;                           // chunk beyond the cache (whole workgroup)
    const int b0 = c * NB;
    // batch tokens whose positions lie in this chunk: t_lo .. t_hi - 1
    const int t_lo = max(0, c * CK - pos0), t_hi = min(T, (c + 1) * CK - pos0);
    const int tn = t_lo + w;                           // this wave's new position (if tn < t_hi)
    const bool has_new = w < t_hi - t_lo;

    // projections (lanes and rows past the batch read zeros), then the cache
    constexpr int QR = 2 * MS;                         // query rows per wave
    const __amdgpu_buffer_rsrc_t rq = vmi_rsrc(a.qkv + (size_t)tok0 * a.stride, (uint32_t)(T * a.stride) * 4u);
    float qv[QR][4], kv[4], vv[4];
    uint32_t qnr[4], knr[4];
#pragma unroll
    for (int i = 0; i < QR; ++i) {
        const int row = w + kChunkWaves * i, t = row / G, h = g * G + row % G;
        const uint32_t base = (uint32_t)(t * a.stride + h * 2 * kHeadDim + lane);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            qv[i][j] = __uint_as_float(vmi_bload_b32(rq, row < R ? (base + 64 * j) * 4u : VMI_OOB, 0));
    }
    {
        const uint32_t kb_ = (uint32_t)(tn * a.stride + a.n_heads * 2 * kHeadDim + g * kHeadDim + lane);
        const uint32_t vb_ = kb_ + (uint32_t)(a.n_kv * kHeadDim);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            kv[j] = __uint_as_float(vmi_bload_b32(rq, has_new ? (kb_ + 64 * j) * 4u : VMI_OOB, 0));
            vv[j] = __uint_as_float(vmi_bload_b32(rq, has_new ? (vb_ + 64 * j) * 4u : VMI_OOB, 0));
        }
    }
    {
        const __amdgpu_buffer_rsrc_t rqn = vmi_rsrc(a.q_norm, kHeadDim * 2u), rkn = vmi_rsrc(a.k_norm, kHeadDim * 2u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            qnr[j] = vmi_bload_b16(rqn, (uint32_t)(lane + 64 * j) * 2u, 0);
            knr[j] = vmi_bload_b16(rkn, (uint32_t)(lane + 64 * j) * 2u, 0);
        }
    }
    asm volatile("" ::: "memory");
    // rotary table while the projections arrive: the angle pos * theta^(-2i/rd)
    // in turns and in double (theta^(-2i/rd) as rope_base^i by repeated
    // squaring), reduced to [-1/2, 1/2] turn, then (cos, sin) of the reduced
    // angle in fp32: within 2e-7 of the exact values at positions up to 2^20,
    // where fp32 rounding of the unreduced angle would move the rotation by
    // up to 1e-3
    {
        const int half = a.rope_dim / 2;
        for (int i = tid; i < T * half; i += kChunkThreads) {
            const int t = i / half, fi = i - t * half;
            double f = 1.0, b = a.rope_base;
            for (int e = fi; e; e >>= 1) {
                if (e & 1) f *= b;
                b *= b;
            }
            const double turns = (double)(pos0 + t) * (f * 0.15915494309189535);  // 1 / (2 pi)
            const float r = (float)((turns - rint(turns)) * 6.283185307179586);
            float sn, cs;
            sincosf(r, &sn, &cs);
            s_cs[t][fi] = make_float2(cs, sn);
        }
    }
    VMI_STAMP(4 + g, 1);
    // the cache blocks: branch-free buffer loads, blocks past the cache
    // reading zeros (a load under a branch would leave every later wait
    // counting as if none of them had been issued)
    const uint32_t head_bytes = (uint32_t)(a.max_len / kKvBlock) * kKvBlockElems * 2u;
    const __amdgpu_buffer_rsrc_t rk = vmi_rsrc(a.k_cache + kv_block(g, a.max_len, 0), head_bytes);
    const __amdgpu_buffer_rsrc_t rv = vmi_rsrc(a.v_cache + kv_block(g, a.max_len, 0), head_bytes);
    vmi_u4 kr[2][8], vr[2][NB];
    const int bw = b0 + w;
    {
        const uint32_t kbase = kKvBlock * bw < L ? (uint32_t)bw * kKvBlockElems * 2u + lane * 16u : VMI_OOB;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) kr[h][kk] = vmi_bload_b128_nt(rk, kbase + (uint32_t)(h * 8 + kk) * 1024u, 0);
    }
    // pieces 2w, 2w + 1 (of 16 x 1 KB) of each extra block's keys
    vmi_u4 kxr[NX > 0 ? NX : 1][2];
#pragma unroll
    for (int x = 0; x < NX; ++x) {
        const int bx = b0 + kChunkWaves + x;
        const uint32_t xbase =
            kKvBlock * bx < L ? (uint32_t)bx * kKvBlockElems * 2u + (uint32_t)(2 * w) * 1024u + lane * 16u : VMI_OOB;
#pragma unroll
        for (int j = 0; j < 2; ++j) kxr[x][j] = vmi_bload_b128_nt(rk, xbase + (uint32_t)j * 1024u, 0);
    }
#pragma unroll
    for (int sb = 0; sb < NB; ++sb) {
        const int bs = b0 + sb;
        const uint32_t vbase =
            kKvBlock * bs < L ? (uint32_t)bs * kKvBlockElems * 2u + (uint32_t)(2 * w) * 1024u + lane * 16u : VMI_OOB;
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) vr[dt][sb] = vmi_bload_b128_nt(rv, vbase + (uint32_t)dt * 1024u, 0);
    }

    __syncthreads();
    VMI_STAMP(4 + g, 2);
    float qn[4], kn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        qn[j] = __uint_as_float(qnr[j] << 16);
        kn[j] = __uint_as_float(knr[j] << 16);
    }
    // the wave's query rows into s_q (rows past the batch: zeros; their
    // projections read as zeros and their table row is a valid one)
    // (up to four rows at once; beyond that two at a time: all of a wave's
    // rows at once would not fit the registers beside the cache operands)
    constexpr int NRB = QR <= 4 ? QR : 2;
    static_assert(QR % NRB == 0, "rows in groups");
#pragma unroll
    for (int i0 = 0; i0 < QR; i0 += NRB) {
        float v2[NRB][4];
        const float2* csr[NRB];
        uint16_t o[NRB][4];
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v2[i][j] = qv[i0 + i][j];
            csr[i] = s_cs[min((w + kChunkWaves * (i0 + i)) / G, T - 1)];
        }
        norm_rope_rows<NRB>(v2, qn, a.eps, csr, a.rope_dim, s_row[w], o);
#pragma unroll
        for (int i = 0; i < NRB; ++i) {
            const int row = w + kChunkWaves * (i0 + i);
            if (row < RP) {
#pragma unroll
                for (int j = 0; j < 4; ++j) s_q[row][lane + 64 * j] = row < R ? o[i][j] : (uint16_t)0;
            }
        }
    }
    VMI_STAMP(4 + g, 7);
    // the new key and value of position pos0 + tn: to the cache (a tree: to
    // the path's rows of tree_kv, committed for the winning path only) and to LDS
    if (has_new) {
        const int pos = pos0 + tn;
        float kv1[1][4] = {{kv[0], kv[1], kv[2], kv[3]}};
        const float2* csk[1] = {s_cs[tn]};
        uint16_t ok[1][4];
        norm_rope_rows<1>(kv1, kn, a.eps, csk, a.rope_dim, s_row[w], ok);
        const uint16_t (&o)[4] = ok[0];
        const size_t blk = kv_block(g, a.max_len, pos);
        const int kt = pos % kKvBlock;
        uint16_t* side = a.tree_kv ? a.tree_kv + ((size_t)(p * a.n_kv + g) * 2 * T + tn) * kHeadDim : nullptr;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int d = lane + 64 * j;
            const uint16_t vb16 = vmi_f32_to_bf16(vv[j]);
            if (side) {
                side[d] = o[j];
                side[(size_t)T * kHeadDim + d] = vb16;
            } else {
                a.k_cache[blk + k_elem(kt, d)] = o[j];
                a.v_cache[blk + v_elem(kt, d)] = vb16;
            }
            s_new[0][tn][d] = o[j];
            s_new[1][tn][d] = vb16;
        }
    }
    VMI_STAMP(4 + g, 8);
    // the extra blocks' keys into LDS (waiting only for those loads: the
    // values, issued after them, keep streaming)
#pragma unroll
    for (int x = 0; x < NX; ++x)
#pragma unroll
        for (int j = 0; j < 2; ++j) s_kx[x][2 * w + j][lane] = kxr[x][j];
    // the last block: values of positions >= L are zeroed (0 * stale could be NaN)
#pragma unroll
    for (int sb = 0; sb < NB; ++sb) {
        const int p0 = kKvBlock * (b0 + sb);
        if (p0 < L && p0 + kKvBlock > L) {
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) vr[dt][sb] = keep_first(vr[dt][sb], L - p0 - 8 * q4);
        }
    }
    VMI_STAMP(4 + g, 9);
    __syncthreads();
    // new keys into the wave's key operands: position kt of the block sits in
    // lanes nl = 4 (kt >> 3) + (kt & 3), tile (kt >> 2) & 1, dims 32 kk + 8 q4 ..
    for (int t = t_lo; t < t_hi; ++t) {
        const int p = pos0 + t;
        if ((p >> 5) != bw) continue;
        const int kt = p & (kKvBlock - 1);
        if (nl == 4 * (kt >> 3) + (kt & 3)) {
            const uint16_t* src = &s_new[0][t][8 * q4];
            if ((kt >> 2) & 1) {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) kr[1][kk] = *reinterpret_cast<const vmi_u4*>(src + 32 * kk);
            } else {
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) kr[0][kk] = *reinterpret_cast<const vmi_u4*>(src + 32 * kk);
            }
        }
    }

    // the extra block of wave w < NX: the batch's new keys into its LDS copy
    // (only this wave reads that copy), as for the registers above
    const bool xw = NX > 0 && w < NX;
    const int bx = b0 + kChunkWaves + w;
    if (xw) {
        for (int t = t_lo; t < t_hi; ++t) {
            const int p = pos0 + t;
            if ((p >> 5) != bx) continue;
            const int kt = p & (kKvBlock - 1);
            if (nl == 4 * (kt >> 3) + (kt & 3)) {
                const uint16_t* src = &s_new[0][t][8 * q4];
                const int hh = (kt >> 2) & 1;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) s_kx[w][8 * hh + kk][lane] = *reinterpret_cast<const vmi_u4*>(src + 32 * kk);
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    VMI_STAMP(4 + g, 3);
    // scores: lane (nl, q4) of tile h holds keys 8 q4 + 4 h + r of block bw
    // (sc) and of block bx (scx, waves w < NX) for query row 16 m + nl
    float sc[MS][8], scx[MS][8];
    auto mask_scale = [&](const vmi_f4& acc0, const vmi_f4& acc1, int p, int last, float (&o)[8]) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o[r] = p + r <= last ? acc0[r] * 0.0625f : -INFINITY;  // 1 / sqrt(256)
            o[4 + r] = p + 4 + r <= last ? acc1[r] * 0.0625f : -INFINITY;
        }
    };
#pragma unroll
    for (int m = 0; m < MS; ++m) {
        vmi_f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
        vmi_f4 ax0 = {0.f, 0.f, 0.f, 0.f}, ax1 = {0.f, 0.f, 0.f, 0.f};
        if (xw) {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const uint4 qv = *reinterpret_cast<const uint4*>(&s_q[16 * m + nl][32 * kk + 8 * q4]);
                const vmi_u4 qb = {qv.x, qv.y, qv.z, qv.w};
                acc0 = vmi_mfma_bf16(kr[0][kk], qb, acc0);
                acc1 = vmi_mfma_bf16(kr[1][kk], qb, acc1);
                ax0 = vmi_mfma_bf16(s_kx[NX > 0 ? w : 0][kk][lane], qb, ax0);
                ax1 = vmi_mfma_bf16(s_kx[NX > 0 ? w : 0][8 + kk][lane], qb, ax1);
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < 8; ++kk) {
                const uint4 qv = *reinterpret_cast<const uint4*>(&s_q[16 * m + nl][32 * kk + 8 * q4]);
                const vmi_u4 qb = {qv.x, qv.y, qv.z, qv.w};
                acc0 = vmi_mfma_bf16(kr[0][kk], qb, acc0);
                acc1 = vmi_mfma_bf16(kr[1][kk], qb, acc1);
            }
        }
        const int row = 16 * m + nl;
        const int last = row < R ? min(L - 1, pos0 + row / G) : -1;  // last visible position
        mask_scale(acc0, acc1, kKvBlock * bw + 8 * q4, last, sc[m]);
        // a wave without an extra block masks it whole (last = -1)
        mask_scale(ax0, ax1, kKvBlock * bx + 8 * q4, xw ? last : -1, scx[m]);
        float mx = sc[m][0];
#pragma unroll
        for (int e = 1; e < 8; ++e) mx = fmaxf(mx, sc[m][e]);
        if (NX > 0) {
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, scx[m][e]);
        }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        if (q4 == 0) s_wm[w][row] = mx;
    }
    __syncthreads();
    VMI_STAMP(4 + g, 4);
    // probabilities against the chunk max, rounded to bf16 (the P.V operand);
    // the row sum adds the rounded values
#pragma unroll
    for (int m = 0; m < MS; ++m) {
        const int row = 16 * m + nl;
        float M = s_wm[0][row];
#pragma unroll
        for (int v = 1; v < kChunkWaves; ++v) M = fmaxf(M, s_wm[v][row]);
        float ls = 0.0f;
        // exp(x - M) as 2^(x log2 e - M log2 e) on the hardware exp2; masked
        // scores (-inf, also in a row with nothing visible) give 0
        const float Ml = M * 1.44269504088896341f;
        auto probs = [&](const float (&sv)[8]) {
            vmi_u4 pk;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x0 = sv[2 * i], x1 = sv[2 * i + 1];
                const float e0 = x0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(x0, 1.44269504088896341f, -Ml));
                const float e1 = x1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(fmaf(x1, 1.44269504088896341f, -Ml));
                const uint32_t u = vmi_pack_bf16x2(e0, e1);
                ls += __uint_as_float(u << 16);
                ls += __uint_as_float(u & 0xffff0000u);
                pk[i] = u;
            }
            return pk;
        };
        s_pa[m][w][lane] = probs(sc[m]);
        if (xw) s_pa[m][NX > 0 ? kChunkWaves + w : 0][lane] = probs(scx[m]);
        ls += __shfl_xor(ls, 16);
        ls += __shfl_xor(ls, 32);
        if (q4 == 0) s_wl[w][row] = ls;
    }
    __syncthreads();
    // new values into the value operands: position 8 q4 + e of block sb is
    // element e of lanes with that q4, dim 32 w + 16 dt + nl
    for (int t = t_lo; t < t_hi; ++t) {
        const int p = pos0 + t, kt = p & (kKvBlock - 1);
        if (q4 != (kt >> 3)) continue;
        const int e = kt & 7;
#pragma unroll
        for (int sb = 0; sb < NB; ++sb) {
            if ((p >> 5) != b0 + sb) continue;
#pragma unroll
            for (int dt = 0; dt < 2; ++dt) {
                const uint32_t nv = s_new[1][t][32 * w + 16 * dt + nl];
#pragma unroll
                for (int ee = 0; ee < 8; ++ee)
                    if (ee == e)
                        vr[dt][sb][ee >> 1] = (ee & 1) ? (vr[dt][sb][ee >> 1] & 0x0000ffffu) | (nv << 16)
                                                       : (vr[dt][sb][ee >> 1] & 0xffff0000u) | nv;
            }
        }
    }
    VMI_STAMP(4 + g, 5);
    // O = P V for dims 32 w + 16 dt + nl; A = P of block sb (written by wave sb)
    const size_t pbase = (((size_t)g * a.nstride + c) * P + p) * RP;  // a chunk holds the rows of every path
#pragma unroll
    for (int m = 0; m < MS; ++m) {
#pragma unroll
        for (int dt = 0; dt < 2; ++dt) {
            vmi_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sb = 0; sb < NB; ++sb) acc = vmi_mfma_bf16(s_pa[m][sb][lane], vr[dt][sb], acc);
            uint16_t* po = a.part_o + (pbase + 16 * m + 4 * q4) * kHeadDim + 32 * w + 16 * dt + nl;
#pragma unroll
            for (int r = 0; r < 4; ++r) po[r * kHeadDim] = (uint16_t)vmi_f32_to_bf16(acc[r]);
        }
    }
    if (tid < RP) {
        float M = s_wm[0][tid], l = s_wl[0][tid];
#pragma unroll
        for (int v = 1; v < kChunkWaves; ++v) {
            M = fmaxf(M, s_wm[v][tid]);
            l += s_wl[v][tid];
        }
        *reinterpret_cast<float2*>(a.part_ml + (pbase + tid) * 2) = make_float2(M, l);
    }
    VMI_STAMP(4 + g, 6);
}

// grid (T * n_heads, 4): one quarter of a head's dims per workgroup.  Chunk c
// is added by slot c % 16 in increasing c and the 16 slots are combined in a
// fixed tree, so the result does not depend on how many chunks a launch has:
// chunks past a query's last position carry weight exactly zero.  Token t
// belongs to path t / span; RP is a path's rows per chunk.
constexpr int kMergeMaxChunks = 2048;
__global__ __launch_bounds__(kAThreads) void k_attn_merge(AttnArgs a, int RP) {
    __shared__ float s_f[kMergeMaxChunks];
    __shared__ float s_red[kAThreads / 64];
    __shared__ float4 s_num[kAThreads / 64][16];
    const int t = blockIdx.x / a.n_heads, h = blockIdx.x % a.n_heads, tid = threadIdx.x;
    const int lane = tid & 63, w = at_wave();
    const int pth = t / a.span, tt = t - pth * a.span;
    const int G = a.n_heads / a.n_kv, g = h / G, row = pth * RP + tt * G + (h % G);
    const int NC = (batch_pos0(a.pos0, a.pos_dev, a.span, a.max_len) + a.span + a.chunk_keys - 1) / a.chunk_keys;
    RP *= a.paths;  // rows per chunk
    // loads in issue order: every chunk's (max, sum) of this row (branch-free,
    // chunks past the cache read nothing), then this lane's first 8 partial
    // outputs, which arrive while the maximum and the denominator form
    constexpr int kMlPer = kMergeMaxChunks / kAThreads;
    const size_t rbase = (size_t)g * a.nstride * RP + row;
    const __amdgpu_buffer_rsrc_t rml = vmi_rsrc(a.part_ml + rbase * 2, (uint32_t)(a.nstride * RP * 2) * 4u);
    const __amdgpu_buffer_rsrc_t rpo =
        vmi_rsrc(a.part_o + rbase * kHeadDim, (uint32_t)(a.nstride * RP) * kHeadDim * 2u);
    uint2 mlr[kMlPer];
#pragma unroll
    for (int i = 0; i < kMlPer; ++i) {
        const int c = tid + kAThreads * i;
        mlr[i] = vmi_bload_b64(rml, c < NC ? (uint32_t)(c * RP * 2) * 4u : VMI_OOB, 0);
    }
    const int slot = 4 * w + (lane >> 4), d0 = 64 * blockIdx.y + 4 * (lane & 15);
    uint2 pv[8];  // four bf16 each
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = slot + 16 * i;
        pv[i] = vmi_bload_b64(rpo, c < NC ? ((uint32_t)(c * RP) * kHeadDim + d0) * 2u : VMI_OOB, 0);
    }
    float M = -INFINITY;
#pragma unroll
    for (int i = 0; i < kMlPer; ++i)
        if (tid + kAThreads * i < NC) M = fmaxf(M, __uint_as_float(mlr[i].x));
    M = vmi_wave_max(M);
    if (lane == 0) s_red[w] = M;
    __syncthreads();
    M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    float den = 0.0f;
#pragma unroll
    for (int i = 0; i < kMlPer; ++i) {
        const int c = tid + kAThreads * i;
        if (c < NC) {
            const float m = __uint_as_float(mlr[i].x);
            const float f = m == -INFINITY ? 0.0f : expf(m - M);
            s_f[c] = f;
            den = fmaf(__uint_as_float(mlr[i].y), f, den);
        }
    }
    den = vmi_wave_sum_canon(den);
    __syncthreads();
    if (lane == 0) s_red[w] = den;
    __syncthreads();
    den = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);

    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    auto add = [&](int c, float vx, float vy, float vz, float vw) {
        const float f = s_f[c];
        acc.x = fmaf(vx, f, acc.x);
        acc.y = fmaf(vy, f, acc.y);
        acc.z = fmaf(vz, f, acc.z);
        acc.w = fmaf(vw, f, acc.w);
    };
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int c = slot + 16 * i;
        if (c < NC) add(c, __uint_as_float(pv[i].x << 16), __uint_as_float(pv[i].x & 0xffff0000u),
                        __uint_as_float(pv[i].y << 16), __uint_as_float(pv[i].y & 0xffff0000u));
    }
    const uint16_t* po = a.part_o + rbase * kHeadDim + d0;  // chunk c at + c * RP * 256
    for (int c0 = slot + 16 * 8; c0 < NC; c0 += 16 * 8) {
        uint2 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = c0 + 16 * i;
            v[i] = c < NC ? *reinterpret_cast<const uint2*>(po + (size_t)c * RP * kHeadDim) : make_uint2(0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int c = c0 + 16 * i;
            if (c < NC)
                add(c, __uint_as_float(v[i].x << 16), __uint_as_float(v[i].x & 0xffff0000u), __uint_as_float(v[i].y << 16),
                    __uint_as_float(v[i].y & 0xffff0000u));
        }
    }
    acc.x += __shfl_xor(acc.x, 16); acc.y += __shfl_xor(acc.y, 16);
    acc.z += __shfl_xor(acc.z, 16); acc.w += __shfl_xor(acc.w, 16);
    acc.x += __shfl_xor(acc.x, 32); acc.y += __shfl_xor(acc.y, 32);
    acc.z += __shfl_xor(acc.z, 32); acc.w += __shfl_xor(acc.w, 32);
    if (lane < 16) s_num[w][lane] = acc;
    __syncthreads();
    if (tid < 16) {
        const float4 n0 = s_num[0][tid], n1 = s_num[1][tid], n2 = s_num[2][tid], n3 = s_num[3][tid];
        const float n[4] = {(n0.x + n1.x) + (n2.x + n3.x), (n0.y + n1.y) + (n2.y + n3.y),
                            (n0.z + n1.z) + (n2.z + n3.z), (n0.w + n1.w) + (n2.w + n3.w)};
        const float* gp = a.qkv + (size_t)t * a.stride + (size_t)h * 2 * kHeadDim + kHeadDim + d0;
        uint32_t out[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float y0 = (den > 0.0f ? n[2 * i] / den : 0.0f) / (1.0f + expf(-gp[2 * i]));
            const float y1 = (den > 0.0f ? n[2 * i + 1] / den : 0.0f) / (1.0f + expf(-gp[2 * i + 1]));
            out[i] = vmi_pack_bf16x2(y0, y1);
        }
        *reinterpret_cast<uint2*>(a.o + ((size_t)t * a.n_heads + h) * kHeadDim + d0) = make_uint2(out[0], out[1]);
    }
}

// ------------------------------------------------------ 4-bit GEMV, MFMA
// out[t][n] = sum_k x[t][k] W[n][k] for 4-bit W with K in {512, 1024, 2048,
// 4096}: 8 waves per workgroup, wave = (16 weight rows, 512 columns), waves
// splitting K meet in LDS in a fixed order.  bf16 MFMAs on exact operands: x
// as it is (each lane reads its 16 bytes of x and puts them in slot order),
// weights as bf16 128 + q (vmi_unpack_u4_bf16_128).  Tokens 0..7 sit in A rows
// 0..7 against the even quantisation group of each 128-column load and in rows
// 8..15 against the odd one, so one MFMA covers both groups and each D lane
// applies its own group's scale:  y = sum_g s_g D_g + (b_g - 128 s_g) X_g with
// X_g the group sum of x.  A token's result does not depend on the batch.
// 8 bf16 values in MFMA operand order: pairs (e, e + 4), the order in which
// vmi_unpack_u4_bf16_128 yields a word's nibbles.
__device__ __forceinline__ uint4 qg_operand_order(const vmi_u4& u) {
    return make_uint4(__builtin_amdgcn_perm(u[2], u[0], 0x05040100u), __builtin_amdgcn_perm(u[2], u[0], 0x07060302u),
                      __builtin_amdgcn_perm(u[3], u[1], 0x05040100u), __builtin_amdgcn_perm(u[3], u[1], 0x07060302u));
}

constexpr int kQ4Waves = 8;
constexpr int kQ4Threads = 64 * kQ4Waves;
constexpr int kQ4Kw = 512;  // columns per wave

// NORM: x is first RMS-normalised (a.norm_w): the workgroup stages the T
// input rows and the norm weights in LDS, wave t computes token t's inverse
// rms in the canonical order (lane L of 64 owns columns [L*cpl, (L+1)*cpl),
// x^2 summed with fmaf in column order, the canonical wave-sum tree, then
// 1/sqrt(ss/K + eps) correctly rounded) and rewrites the row as
// bf16((x * inv) * w) in place - what k_rms_rows writes - and every wave reads
// its operands from there.
constexpr int kQ4MaxK = 2048;  // widest K the NORM form stages

// RT: weight rows per wave tile, 16, or 8 where 16-row tiles would leave
// half the CUs idle (lanes 8..15 then repeat rows 0..7: the same addresses in
// the same load, and MFMA columns 8..15 that are not stored).
template <bool NORM, int RT, int NW>
__global__ __launch_bounds__(NW * 64) void k_qgemv4(QgArgs a) {
    static_assert(RT == 8 || RT == 16, "row tile");
    static_assert(NW == kQ4Waves || (NW == 12 && NORM), "8 waves, or 12 for the normalising form");
    constexpr int NT = NW * 64;
    __shared__ float s_part[NW][16][kQgMaxT];
    const int T = a.T, K = a.K, G = K / 64;
    const int tid = threadIdx.x, lane = tid & 63, w = at_wave();
    const int nl = lane & 15, q4 = lane >> 4;
    constexpr int kid = NORM ? 3 : 2;  // timeline kernel id of the form
    VMI_STAMP(kid, 0);
    VMI_STAMP_HWID(kid, 4);
    // every argument read below in SGPRs at once: one wait for the argument
    // block (fields read lazily, under the matrix branches, cost a round trip
    // each before the first load could issue)
    asm volatile("" ::"s"(a.x), "s"(a.m[0].w), "s"(a.m[0].s), "s"(a.m[0].b), "s"(a.m[1].w), "s"(a.m[1].s),
                 "s"(a.m[1].b), "s"(a.m[2].w), "s"(a.m[2].s), "s"(a.m[2].b));
    asm volatile("" ::"s"(a.rows[0]), "s"(a.rows[1]), "s"(a.nrows), "s"(a.residual), "s"(a.out_bf16), "s"(a.out),
                 "s"(a.out_stride), "s"(T), "s"(K));
    const int lks = __builtin_ctz((unsigned)K) - 9;  // K / kQ4Kw = 1 << lks (K is 512, 1024, 2048 or 4096)
    const int ks = 1 << lks, tiles = NW >> lks;
    const int tile = w >> lks, kw = w & (ks - 1);
    const int n = (blockIdx.x * tiles + tile) * RT + (nl & (RT - 1));
    const int nn = n < a.nrows ? n : a.nrows - 1;
    // matrix of row nn, selected from the kernel arguments by value (an
    // indexed argument would be a dependent vector load before the weights)
    int mi = 0, r = nn;
    if (r >= a.rows[0]) {
        r -= a.rows[0];
        mi = 1;
        if (r >= a.rows[1]) {
            r -= a.rows[1];
            mi = 2;
        }
    }
    vmi_qmat M;
    M.w = mi == 0 ? a.m[0].w : mi == 1 ? a.m[1].w : a.m[2].w;
    M.s = mi == 0 ? a.m[0].s : mi == 1 ? a.m[1].s : a.m[2].s;
    M.b = mi == 0 ? a.m[0].b : mi == 1 ? a.m[1].b : a.m[2].b;
    // A operands: token tk, columns kw*512 + 128 m + 32 q4 + 8 j .. + 7
    const int tk = nl & 7;
    const bool xreal = ((q4 < 2) == (nl < 8)) && tk < T;
    const uint4* xr;  // the lane's operand words in LDS (set below)
    // Without the norm, each wave reads its 512-column slice of the T input
    // rows first, whole 1 KB rows per load (lane L: 16 bytes at 16 L), and
    // puts it in operand order through LDS below.  The operand order itself
    // (16 bytes at 64-byte steps across the lanes, 16 loads a lane) touched
    // eight times as many cache lines and was what the CU's load pipeline
    // spent its time on.
    vmi_u4 xv[kQgMaxT];
    if constexpr (!NORM) {
        const __amdgpu_buffer_rsrc_t rx = vmi_rsrc(a.x, (uint32_t)(T * K) * 2u);
#pragma unroll
        for (int i = 0; i < kQgMaxT; ++i)
            if (i < T) xv[i] = vmi_bload_b128(rx, (uint32_t)((i * K + kw * kQ4Kw) * 2 + lane * 16), 0);
        asm volatile("" ::: "memory");
    }
    constexpr int NXW = NORM ? (kQgMaxT * kQ4MaxK / 8 + NT - 1) / NT : 1;
    vmi_u4 xw[NXW], nw;
    if constexpr (NORM) {
        // the T input rows and the norm weights as 16-byte words, first: the
        // norm waits for them, and loads complete in issue order
        const __amdgpu_buffer_rsrc_t rx = vmi_rsrc(a.x, (uint32_t)(T * K / 8) * 16u);
        const __amdgpu_buffer_rsrc_t rn = vmi_rsrc(a.norm_w, (uint32_t)(K / 8) * 16u);
#pragma unroll
        for (int d = 0; d < NXW; ++d) xw[d] = vmi_bload_b128(rx, (uint32_t)(tid + NT * d) * 16u, 0);
        nw = vmi_bload_b128(rn, (uint32_t)tid * 16u, 0);
        asm volatile("" ::: "memory");
    }
    // Every wave's input loads are issued before any wave's weight loads: a
    // CU returns vector loads in issue order, so a wave that issued its
    // input behind another wave's weights would wait for those weights
    // (waves 4..7 had their x 1.6 us after waves 0..3).  The barrier does
    // not wait for the loads themselves.  The normalising form goes without:
    // its input words are two whole-row loads a thread, and it measured
    // slightly faster without the barrier.
    if constexpr (!NORM) __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint4* wrow = reinterpret_cast<const uint4*>(M.w + (size_t)r * (K / 8));
    uint4 wv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {  // weights are read once per step: nontemporal
        const vmi_u4 u = __builtin_nontemporal_load(reinterpret_cast<const vmi_u4*>(wrow) + kw * 16 + 4 * m + q4);
        wv[m] = make_uint4(u[0], u[1], u[2], u[3]);
    }
    const vmi_u4 su = __builtin_nontemporal_load(reinterpret_cast<const vmi_u4*>(M.s + (size_t)r * G + kw * 8));
    const vmi_u4 bu = __builtin_nontemporal_load(reinterpret_cast<const vmi_u4*>(M.b + (size_t)r * G + kw * 8));
    const uint4 sv = make_uint4(su[0], su[1], su[2], su[3]), bv = make_uint4(bu[0], bu[1], bu[2], bu[3]);
    // the residual of this thread's output (first pass of the final loop) as
    // raw bf16 bits, issued now so that its latency overlaps the weights'; a
    // branch-free buffer load whose value is first used at the end, so no
    // wait on it (and on everything issued before it) lands here
    // outputs i = (tile, row, token) with the token in the low three bits
    // (kQgMaxT = 8 slots, those past T idle): shifts, not divisions by T
    static_assert(kQgMaxT == 8, "three token bits");
    constexpr int LRT = RT == 16 ? 4 : 3;
    const int nout = tiles * RT * kQgMaxT;
    // (unconditional: without a residual the range is empty and every lane
    // reads zero without touching memory)
    const __amdgpu_buffer_rsrc_t rres =
        vmi_rsrc(a.residual, a.out_bf16 && a.residual ? (uint32_t)((size_t)T * a.out_stride * 2) : 0u);
    const int row0 = (blockIdx.x * tiles + (tid >> (3 + LRT))) * RT + ((tid >> 3) & (RT - 1)), t0 = tid & 7;
    const uint32_t res0 = vmi_bload_b16(
        rres, tid < nout && t0 < T && row0 < a.nrows ? (uint32_t)(((size_t)t0 * a.out_stride + row0) * 2) : VMI_OOB, 0);
    asm volatile("" ::: "memory");
    VMI_STAMP(kid, 5);
    if constexpr (!NORM) {
        // the wave's slice into its own LDS rows (padded by 16 bytes against
        // bank conflicts between tokens); the same wave reads it back in
        // operand order below
        // (row kQgMaxT stays zero: the operand row of lanes outside the batch)
        __shared__ uint4 s_xw[NW][kQgMaxT + 1][kQ4Kw / 8 + 1];
        s_xw[w][kQgMaxT][lane] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int i = 0; i < kQgMaxT; ++i)
            if (i < T) s_xw[w][i][lane] = qg_operand_order(xv[i]);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        xr = &s_xw[w][xreal ? tk : kQgMaxT][4 * q4];
    }
    if constexpr (NORM) {
        // the rows into LDS, wave t normalises token t there, every wave then
        // reads its operands (the weights keep streaming meanwhile)
        // (row kQgMaxT: zeros, the operand row of lanes outside the batch)
        __shared__ uint4 s_xn[(kQgMaxT + 1) * kQ4MaxK / 8];
        __shared__ uint4 s_nw[kQ4MaxK / 8];
        const int nxw = T * K / 8, nnw = K / 8;
        if (tid < nnw) s_xn[kQgMaxT * (K / 8) + tid] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int d = 0; d < NXW; ++d) {
            const int i = tid + NT * d;
            if (i < nxw) s_xn[i] = make_uint4(xw[d][0], xw[d][1], xw[d][2], xw[d][3]);
        }
        if (tid < nnw) s_nw[tid] = make_uint4(nw[0], nw[1], nw[2], nw[3]);
        __shared__ float s_inv[kQgMaxT];
        __syncthreads();
        if (w < T) {
            const int cpl = K / 64, nv = cpl / 8;
            const uint4* row = s_xn + (size_t)w * (K / 8) + lane * nv;
            float ss = 0.0f;
            for (int v = 0; v < nv; ++v) {
                float f[8];
                bf16x8f(row[v], f);
#pragma unroll
                for (int i = 0; i < 8; ++i) ss = fmaf(f[i], f[i], ss);
            }
            ss = vmi_wave_sum_canon(ss);
            if (lane == 0) s_inv[w] = __fdiv_rn(1.0f, __fsqrt_rn(ss * (1.0f / (float)K) + a.eps));
        }
        __syncthreads();
        // every thread rewrites its words of the rows in place
#pragma unroll
        for (int d = 0; d < NXW; ++d) {
            const int i = tid + NT * d;
            if (i < nxw) {
                const float inv = s_inv[i / (K / 8)];
                float f[8], g[8];
                bf16x8f(s_xn[i], f);
                bf16x8f(s_nw[i % (K / 8)], g);
                // in MFMA operand order: pairs (e, e + 4), the weight unpack's order
                uint32_t o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    o[e] = vmi_pack_bf16x2((f[e] * inv) * g[e], (f[e + 4] * inv) * g[e + 4]);
                s_xn[i] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
        __syncthreads();
        xr = s_xn + (size_t)(xreal ? tk : kQgMaxT) * (K / 8) + kw * (kQ4Kw / 8) + 4 * q4;
    }
    VMI_STAMP(kid, 6);
    // the lane's operand words from LDS, already in operand order (uint4
    // 16 m + 4 q4 + j of its token's slice; lanes outside the batch read the
    // zero row)
    vmi_u4 ax[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint4 u = xr[16 * m + j];
            ax[m][j] = vmi_u4{u.x, u.y, u.z, u.w};
        }
    const int par = q4 >> 1;
    VMI_STAMP(kid, 7);
    const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w}, bw[4] = {bv.x, bv.y, bv.z, bv.w};
    const vmi_f4 zf = {0.f, 0.f, 0.f, 0.f};
    // X_g, the group sums of x, by the matrix core: against an all-ones B,
    // D row 4 q4 + e (token 4 (q4 & 1) + e, group 2m + par) is the sum of the
    // 64 values of that token's group in every column, so each lane gets the
    // sums its own outputs need (zero for rows outside the batch)
    const vmi_u4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
    vmi_f4 xg[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const uint32_t ww[4] = {wv[m].x, wv[m].y, wv[m].z, wv[m].w};
        vmi_f4 d = zf, xd = zf;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d = vmi_mfma_bf16(ax[m][j], vmi_unpack_u4_bf16_128(ww[j]), d);
            xd = vmi_mfma_bf16(ax[m][j], ones, xd);
        }
        xg[m] = xd;
        const float sc = __uint_as_float(par ? (sw[m] & 0xffff0000u) : (sw[m] << 16));
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(sc, d[e], acc[e]);
    }
    VMI_STAMP(kid, 1);
    // (b_g - 128 s_g) X_g over the groups of this lane's parity
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float sc = __uint_as_float(par ? (sw[m] & 0xffff0000u) : (sw[m] << 16));
        const float bi = __uint_as_float(par ? (bw[m] & 0xffff0000u) : (bw[m] << 16));
        const float c = fmaf(-128.0f, sc, bi);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[e] = fmaf(c, xg[m][e], acc[e]);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], 32);
    if (q4 < 2) {
#pragma unroll
        for (int e = 0; e < 4; ++e) s_part[w][nl][4 * q4 + e] = acc[e];
    }
    __syncthreads();
    VMI_STAMP(kid, 2);
    for (int i = tid; i < nout; i += NT) {
        const int tl = i >> (3 + LRT), rr = (i >> 3) & (RT - 1), t = i & 7;
        if (t >= T) continue;
        float y = s_part[tl * ks][rr][t];
        for (int k2 = 1; k2 < ks; ++k2) y += s_part[tl * ks + k2][rr][t];
        const int row = (blockIdx.x * tiles + tl) * RT + rr;
        if (row < a.nrows) {
            if (a.out) a.out[(size_t)t * a.out_stride + row] = y;
            if (a.out_bf16) {
                const float res = !a.residual ? 0.0f
                                  : i == tid ? __uint_as_float(res0 << 16)
                                             : vmi_bf16_to_f32(a.residual[(size_t)t * a.out_stride + row]);
                a.out_bf16[(size_t)t * a.out_stride + row] = vmi_f32_to_bf16(y + res);
            }
        }
    }
    VMI_STAMP(kid, 3);
}

// ------------------------------------------------------------------ host
// Keys are split into chunks at fixed absolute positions, so a query's result
// does not depend on how many tokens share its batch.  Upper bound of the
// chunk count (256-key chunks), for buffer sizes:
int attn_chunks(int L) { return (L + kChunkKeys - 1) / kChunkKeys; }

// Blocks per chunk beyond 8 for a cache of max_len positions: the fewest that
// give every chunk of every kv head a CU of its own (one chunk workgroup per
// CU), at most kMaxExtraBlocks.  A function of the cache capacity and the
// device alone, so every call on one cache (any batch size, a tree or a
// single path) splits the keys alike.
int attn_extra_blocks(int max_len, int n_kv) {
    const int ncu = vmi::device_cus();
    const int blocks = max_len / kKvBlock;  // per kv head
    for (int nx = 0; nx < kMaxExtraBlocks; ++nx)
        if ((long)n_kv * ((blocks + kChunkWaves + nx - 1) / (kChunkWaves + nx)) <= ncu) return nx;
    return kMaxExtraBlocks;
}

struct AttnLayout {
    size_t status, xn, qkv, part_o, part_ml, o, bytes;
};

AttnLayout attn_layout(int T, int H, int n_heads, int n_kv, int max_len, int paths = 1) {
    AttnLayout L{};
    size_t off = 0;
    auto take = [&](size_t b) {
        const size_t o = off;
        off += vmi::align256(b);
        return o;
    };
    const int RP = paths * 16 * ((T / paths * (n_heads / n_kv) + 15) / 16);
    const int stride = n_heads * 2 * kHeadDim + 2 * n_kv * kHeadDim;
    L.status = take(4);
    L.xn = take((size_t)T * H * 2);
    L.qkv = take((size_t)T * stride * 4);
    const int nc = attn_chunks(max_len);
    L.part_o = take((size_t)n_kv * nc * RP * kHeadDim * 2);
    L.part_ml = take((size_t)n_kv * nc * RP * 2 * 4);
    L.o = take((size_t)T * n_heads * kHeadDim * 2);
    L.bytes = off;
    return L;
}

bool qm_ok(const vmi_qmat& m) { return vmi::qmat_ok(m); }

}  // namespace

hipError_t vmi::launch_qgemv(const QgemvCall& q0, hipStream_t s) {
    if (q0.T > kQgMaxT) {
        // pieces of up to kQgMaxT tokens: a token's result does not depend on its batch
        for (int t0 = 0; t0 < q0.T; t0 += kQgMaxT) {
            QgemvCall c = q0;
            c.T = q0.T - t0 < kQgMaxT ? q0.T - t0 : kQgMaxT;
            c.x = q0.x + (size_t)t0 * q0.K;
            if (c.out) c.out = q0.out + (size_t)t0 * q0.out_stride;
            if (c.out_bf16) c.out_bf16 = q0.out_bf16 + (size_t)t0 * q0.out_stride;
            if (c.residual) c.residual = q0.residual + (size_t)t0 * q0.out_stride;
            const hipError_t e = launch_qgemv(c, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const QgemvCall& q = q0;
    const int ks = q.K / kQ4Kw;
    uintptr_t sb_align = 0;  // the MFMA kernel reads 8 scales / biases as one 16-byte load
    for (int i = 0; i < 3; ++i)
        if (q.rows[i] > 0 || i == 0)
            sb_align |= reinterpret_cast<uintptr_t>(q.m[i].s) | reinterpret_cast<uintptr_t>(q.m[i].b);
    if (q.norm_w && !qgemv_fuses_norm(q)) return hipErrorInvalidValue;
    if (q.bits == 4 && q.K % kQ4Kw == 0 && ks <= kQ4Waves && kQ4Waves % ks == 0 && !(sb_align & 15)) {
        // 8-row tiles when 16-row tiles fill at most half the CUs and 8-row
        // ones still give each workgroup a CU of its own
        const int tiles = kQ4Waves / ks;
        const int wg16 = (q.nrows + 16 * tiles - 1) / (16 * tiles), wg8 = (q.nrows + 8 * tiles - 1) / (8 * tiles);
        const int ncu = vmi::device_cus();
        const bool rt8 = 2 * wg16 <= ncu && wg8 <= ncu;
        // 12-wave workgroups of three 16-row tiles (normalising form) when the
        // 8-wave ones would put two workgroups on some CU and three tiles per
        // workgroup give every workgroup a CU of its own (9,216 and 12,288
        // rows at K = 2048: 192 and 256 workgroups instead of 288 and 384)
        const int tiles12 = 12 / ks, wg12 = (q.nrows + 16 * tiles12 - 1) / (16 * tiles12);
        const bool w12 = q.norm_w && !rt8 && 12 % ks == 0 && wg16 > ncu && wg12 <= ncu;
        const dim3 grid(rt8 ? wg8 : w12 ? wg12 : wg16);
        if (q.norm_w) {
            if (rt8)
                hipLaunchKernelGGL((k_qgemv4<true, 8, kQ4Waves>), grid, dim3(kQ4Threads), 0, s, q);
            else if (w12)
                hipLaunchKernelGGL((k_qgemv4<true, 16, 12>), grid, dim3(12 * 64), 0, s, q);
            else
                hipLaunchKernelGGL((k_qgemv4<true, 16, kQ4Waves>), grid, dim3(kQ4Threads), 0, s, q);
        } else {
            if (rt8)
                hipLaunchKernelGGL((k_qgemv4<false, 8, kQ4Waves>), grid, dim3(kQ4Threads), 0, s, q);
            else
                hipLaunchKernelGGL((k_qgemv4<false, 16, kQ4Waves>), grid, dim3(kQ4Threads), 0, s, q);
        }
    } else {
        const size_t lds = (size_t)q.T * q.K * 2;
        hipLaunchKernelGGL(k_qgemv, dim3((q.nrows + 3) / 4), dim3(kAThreads), lds, s, q);
    }
    return hipGetLastError();
}

hipError_t vmi::launch_rmsnorm(const uint16_t* x, const uint16_t* w, float eps, int T, int H, uint16_t* out,
                               hipStream_t s) {
    RmsArgs ra{x, w, eps, T, H, out, nullptr, 0, nullptr, H};
    hipLaunchKernelGGL(k_rms_rows, dim3((T + 3) / 4), dim3(kAThreads), 0, s, ra);
    return hipGetLastError();
}

bool vmi::qgemv_fuses_norm(const QgemvCall& q) {
    uintptr_t sb_align = 0;
    for (int i = 0; i < 3; ++i)
        if (q.rows[i] > 0 || i == 0)
            sb_align |= reinterpret_cast<uintptr_t>(q.m[i].s) | reinterpret_cast<uintptr_t>(q.m[i].b);
    return q.bits == 4 && (q.K == 512 || q.K == 1024 || q.K == kQ4MaxK) && !(sb_align & 15) &&
           !(reinterpret_cast<uintptr_t>(q.norm_w) & 15);
}

bool vmi::qmat_ok(const vmi_qmat& m) {
    return m.w && m.s && m.b && !(reinterpret_cast<uintptr_t>(m.w) & 15);
}

extern "C" int vmi_qgemv(const uint16_t* x, int T, int K, vmi_qmat w, int N, int bits, int group, float* out,
                         const uint16_t* residual, uint16_t* out_bf16, void* stream) {
    vmi::clear_error();
    if (T <= 0 || T > kQgMaxBatch) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d must be in [1, %d]", T, kQgMaxBatch);
    if (K <= 0 || K % 64 || N <= 0) return vmi::fail(VMI_ERR_INVALID, "K=%d (multiple of 64) N=%d", K, N);
    if ((size_t)(T < kQgMaxT ? T : kQgMaxT) * K * 2 > 65536)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "K=%d too wide for %d tokens", K, T);
    if ((bits != 4 && bits != 8) || group != 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "bits=%d group=%d", bits, group);
    if (!x || !qm_ok(w) || (!out && !out_bf16)) return vmi::fail(VMI_ERR_INVALID, "null x/weights/out");
    if ((reinterpret_cast<uintptr_t>(x) & 15)) return vmi::fail(VMI_ERR_INVALID, "x must be 16-byte aligned");
    QgArgs q{};
    q.x = x; q.T = T; q.K = K; q.bits = bits;
    q.m[0] = w; q.m[1] = w; q.m[2] = w;
    q.rows[0] = N; q.rows[1] = 0; q.rows[2] = 0; q.nrows = N;
    q.out = out; q.out_stride = N; q.residual = residual; q.out_bf16 = out_bf16;
    const hipError_t e = vmi::launch_qgemv(q, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_qgemv launch");
}

extern "C" size_t vmi_attention_layer_workspace_bytes(int T, int hidden, int n_heads, int n_kv_heads, int max_len) {
    if (T <= 0 || hidden <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || max_len <= 0) return 0;
    return attn_layout(T, hidden, n_heads, n_kv_heads, max_len).bytes;
}

extern "C" size_t vmi_attention_tree_workspace_bytes(int paths, int span, int hidden, int n_heads, int n_kv_heads,
                                                     int max_len) {
    if (paths <= 0 || span <= 0 || hidden <= 0 || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads ||
        max_len <= 0)
        return 0;
    return attn_layout(paths * span, hidden, n_heads, n_kv_heads, max_len, paths).bytes;
}

namespace {

// The attention block over `paths` sequences of `span` tokens that share the
// cache up to pos0 (one path: the verify batch; several: a draft tree, new
// keys/values to tree_kv instead of the cache).
int attention_impl(const vmi_attn_layer_desc* desc, const uint16_t* x, int paths, int span, int pos0,
                   const int32_t* pos_device, uint16_t* k_cache, uint16_t* v_cache, int max_len, uint16_t* tree_kv,
                   uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
    if (!desc) return vmi::fail(VMI_ERR_INVALID, "null desc");
    const vmi_attn_layer_desc& D = *desc;
    const int T = paths * span;
    if (span <= 0 || span > kQgMaxT) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d must be in [1, %d]", span, kQgMaxT);
    if (paths <= 0 || T > kQgMaxBatch)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "paths=%d x span=%d exceeds %d tokens", paths, span, kQgMaxBatch);
    if (D.head_dim != kHeadDim) return vmi::fail(VMI_ERR_UNSUPPORTED, "head_dim=%d (256 only)", D.head_dim);
    if (D.n_heads <= 0 || D.n_kv_heads <= 0 || D.n_heads % D.n_kv_heads)
        return vmi::fail(VMI_ERR_INVALID, "n_heads=%d n_kv_heads=%d", D.n_heads, D.n_kv_heads);
    const int G = D.n_heads / D.n_kv_heads;
    if (span * G > 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "T * heads per kv head = %d exceeds 64", span * G);
    if (D.hidden % 512 || D.hidden > 4096) return vmi::fail(VMI_ERR_UNSUPPORTED, "hidden=%d", D.hidden);
    const int Tp = T < kQgMaxT ? T : kQgMaxT;  // tokens of one GEMV launch
    if (D.n_heads * kHeadDim * Tp * 2 > 65536 || D.hidden * Tp * 2 > 65536)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "T too large for the projection GEMV");
    if (D.rope_dim < 0 || D.rope_dim > kHeadDim || D.rope_dim % 2) return vmi::fail(VMI_ERR_INVALID, "rope_dim=%d", D.rope_dim);
    if ((D.bits != 4 && D.bits != 8) || D.group != 64) return vmi::fail(VMI_ERR_UNSUPPORTED, "bits=%d group=%d", D.bits, D.group);
    if (span > max_len || (!pos_device && (pos0 < 0 || pos0 + span > max_len)))
        return vmi::fail(VMI_ERR_INVALID, "pos0=%d T=%d max_len=%d", pos0, span, max_len);
    if (max_len % kKvBlock) return vmi::fail(VMI_ERR_INVALID, "max_len=%d must be a multiple of %d", max_len, kKvBlock);
    if (attn_chunks(max_len) > kMergeMaxChunks)
        return vmi::fail(VMI_ERR_UNSUPPORTED, "max_len=%d exceeds %d", max_len, kMergeMaxChunks * kChunkKeys);
    if (!x || !out || !k_cache || !v_cache || !D.input_norm || !D.q_norm || !D.k_norm)
        return vmi::fail(VMI_ERR_INVALID, "null x/out/cache/norm weights");
    if (!qm_ok(D.q_proj) || !qm_ok(D.k_proj) || !qm_ok(D.v_proj) || !qm_ok(D.o_proj))
        return vmi::fail(VMI_ERR_INVALID, "projection weights must be non-null and 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(k_cache) |
         reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(D.input_norm)) & 15)
        return vmi::fail(VMI_ERR_INVALID, "x, out, caches and norm weight must be 16-byte aligned");
    const AttnLayout L = attn_layout(T, D.hidden, D.n_heads, D.n_kv_heads, max_len, paths);
    if (!workspace || workspace_bytes < L.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", L.bytes, workspace_bytes);
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    uint16_t* xn = reinterpret_cast<uint16_t*>(ws + L.xn);
    float* qkv = reinterpret_cast<float*>(ws + L.qkv);
    uint16_t* ob = reinterpret_cast<uint16_t*>(ws + L.o);
    const int stride = D.n_heads * 2 * kHeadDim + 2 * D.n_kv_heads * kHeadDim;
    hipStream_t s = static_cast<hipStream_t>(stream);

    // input RMSNorm inside the projection when the GEMV can take it, else its own kernel
    QgArgs q{};
    q.x = x; q.T = T; q.K = D.hidden; q.bits = D.bits;
    q.m[0] = D.q_proj; q.m[1] = D.k_proj; q.m[2] = D.v_proj;
    q.rows[0] = D.n_heads * 2 * kHeadDim; q.rows[1] = D.n_kv_heads * kHeadDim; q.rows[2] = D.n_kv_heads * kHeadDim;
    q.nrows = stride; q.out = qkv; q.out_stride = stride;
    q.norm_w = D.input_norm; q.eps = D.norm_eps;
    if (!vmi::qgemv_fuses_norm(q)) {
        RmsArgs ra{x, D.input_norm, D.norm_eps, T, D.hidden, xn, nullptr, 0, nullptr, D.hidden};
        hipLaunchKernelGGL(k_rms_rows, dim3((T + 3) / 4), dim3(kAThreads), 0, s, ra);
        q.x = xn;
        q.norm_w = nullptr;
    }
    hipError_t e = vmi::launch_qgemv(q, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "qkv projection launch");

    AttnArgs at{};
    at.qkv = qkv; at.stride = stride; at.q_norm = D.q_norm; at.k_norm = D.k_norm;
    at.rope_dim = D.rope_dim; at.eps = D.norm_eps;
    at.rope_base = D.rope_dim ? pow((double)D.rope_theta, -2.0 / (double)D.rope_dim) : 1.0;
    at.k_cache = k_cache; at.v_cache = v_cache;
    at.T = T; at.n_heads = D.n_heads; at.n_kv = D.n_kv_heads; at.pos0 = pos0; at.pos_dev = pos_device;
    at.paths = paths; at.span = span; at.tree_kv = tree_kv;
    at.status = reinterpret_cast<uint32_t*>(ws + L.status);
    at.max_len = max_len;
    const int NX = attn_extra_blocks(max_len, D.n_kv_heads);
    at.chunk_keys = (kChunkWaves + NX) * kKvBlock;
    at.nstride = (max_len + at.chunk_keys - 1) / at.chunk_keys;  // <= attn_chunks(max_len): the layout's bound
    // with the position on the device every chunk of the capacity is launched; those past the cache exit
    const int grid_chunks = pos_device ? at.nstride : (pos0 + span + at.chunk_keys - 1) / at.chunk_keys;
    at.chunks = grid_chunks;
    at.part_o = reinterpret_cast<uint16_t*>(ws + L.part_o);
    at.part_ml = reinterpret_cast<float*>(ws + L.part_ml);
    at.o = ob;
    const int MS = (span * G + 15) / 16;
    const dim3 ag(paths == 1 ? grid_chunks : (grid_chunks + 7) / 8 * 8 * paths, D.n_kv_heads);
    static_assert(kMaxExtraBlocks == 2, "the launch below covers NX = 0..2");
    auto chunk_kernel = [&](auto ms) {
        constexpr int M = decltype(ms)::value;
        if (NX == 0)
            hipLaunchKernelGGL((k_attn_chunk<M, 0>), ag, dim3(kChunkThreads), 0, s, at);
        else if (NX == 1)
            hipLaunchKernelGGL((k_attn_chunk<M, 1>), ag, dim3(kChunkThreads), 0, s, at);
        else
            hipLaunchKernelGGL((k_attn_chunk<M, 2>), ag, dim3(kChunkThreads), 0, s, at);
    };
    switch (MS) {
        case 1: chunk_kernel(std::integral_constant<int, 1>{}); break;
        case 2: chunk_kernel(std::integral_constant<int, 2>{}); break;
        case 3: chunk_kernel(std::integral_constant<int, 3>{}); break;
        default: chunk_kernel(std::integral_constant<int, 4>{}); break;
    }
    hipLaunchKernelGGL(k_attn_merge, dim3(T * D.n_heads, 4), dim3(kAThreads), 0, s, at, 16 * MS);

    QgArgs o{};
    o.x = ob; o.T = T; o.K = D.n_heads * kHeadDim; o.bits = D.bits;
    o.m[0] = D.o_proj; o.m[1] = D.o_proj; o.m[2] = D.o_proj;
    o.rows[0] = D.hidden; o.rows[1] = 0; o.rows[2] = 0; o.nrows = D.hidden;
    o.out = nullptr; o.out_stride = D.hidden; o.residual = x; o.out_bf16 = out;
    e = vmi::launch_qgemv(o, s);
    if (e != hipSuccess) return vmi::hip_fail(e, "o_proj launch");
    return VMI_OK;
}

}  // namespace

extern "C" int vmi_attention_layer(const vmi_attn_layer_desc* desc, const uint16_t* x, int T, int pos0,
                                   const int32_t* pos_device, uint16_t* k_cache, uint16_t* v_cache, int max_len, uint16_t* out,
                                   void* workspace, size_t workspace_bytes, void* stream) {
    vmi::clear_error();
    return attention_impl(desc, x, 1, T, pos0, pos_device, k_cache, v_cache, max_len, nullptr, out, workspace,
                          workspace_bytes, stream);
}

extern "C" int vmi_attention_tree(const vmi_attn_layer_desc* desc, const uint16_t* x, int paths, int span, int pos0,
                                  const int32_t* pos_device, const uint16_t* k_cache, const uint16_t* v_cache,
                                  int max_len, uint16_t* tree_kv, uint16_t* out, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    vmi::clear_error();
    if (paths < 1 || !tree_kv) return vmi::fail(VMI_ERR_INVALID, "paths=%d tree_kv=%p", paths, (void*)tree_kv);
    // the caches are only read: every path's new keys and values go to tree_kv
    return attention_impl(desc, x, paths, span, pos0, pos_device, const_cast<uint16_t*>(k_cache),
                          const_cast<uint16_t*>(v_cache), max_len, tree_kv, out, workspace, workspace_bytes, stream);
}

extern "C" int vmi_rmsnorm(const uint16_t* x, const int32_t* ids, int rows, int T, int hidden, const uint16_t* weight,
                           float eps, uint16_t* out, int out_stride, uint32_t* status, void* stream) {
    vmi::clear_error();
    if (T <= 0 || hidden <= 0 || hidden % 512) return vmi::fail(VMI_ERR_UNSUPPORTED, "T=%d hidden=%d", T, hidden);
    if (!x || !out) return vmi::fail(VMI_ERR_INVALID, "null x/out");
    if (ids && rows <= 0) return vmi::fail(VMI_ERR_INVALID, "rows=%d", rows);
    if (out_stride < hidden || out_stride % 8) return vmi::fail(VMI_ERR_INVALID, "out_stride=%d", out_stride);
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight) | reinterpret_cast<uintptr_t>(out)) & 15)
        return vmi::fail(VMI_ERR_INVALID, "x, weight and out must be 16-byte aligned");
    RmsArgs ra{x, weight, eps, T, hidden, out, ids, rows, status, out_stride};
    hipLaunchKernelGGL(k_rms_rows, dim3((T + 3) / 4), dim3(kAThreads), 0, static_cast<hipStream_t>(stream), ra);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_rms_rows launch");
}

#ifdef VMI_TIMELINE
// Tuning builds only: where the kernels of this file record their stamps.
extern "C" int vmi_timeline_set_attn(void* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(vmi_tl_buf), &buf, sizeof(buf)) == hipSuccess ? VMI_OK : VMI_ERR_HIP;
}
#endif
