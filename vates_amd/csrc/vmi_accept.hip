// Acceptance of a speculative verify step, on the device.
//
// k_accept_greedy   longest-prefix acceptance (generate.py:338-351) of one
//                   draft chain, or of P draft paths with the winner chosen as
//                   the longest match, ties to the lower path (generate.py:383),
//                   and the emission rules of generate.py:819, :850-856.
// Speculative sampling (Leviathan et al. 2023, Algorithm 1): keep draft d_i
// when u_i q(d_i) <= p(d_i), else draw from norm(max(0, p - q)); a bonus token
// from p_K when every draft is kept.  p and q are temperature / top-p
// transforms of the target and draft logits.  The same machinery samples one
// token per row (the drafter's sampler).  One launch (k_sd_fused): each
// distribution's vocabulary is split over NB resident workgroups, which meet
// at per-distribution arrival counters between the phases (maxima, masses and
// level-1 histogram, level-2 and level-3 histograms of a three-level radix
// select of the top-p threshold, the draw).  Histograms are integer sums
// (global atomics), so their value does not depend on arrival order.
//
// Every probability is an integer mass (W_j = floor(2^31 2^z), z =
// (l_j - max l) / temperature * log2 e, 2^z from a fixed fp32 polynomial), so
// sums are exact in any order and the results are bit-identical to the CPU
// oracle; decisions use IEEE double operations only.  Uniforms come from
// Philox4x32-10 (key = seed, counter = (offset, position, 0x5A3D1E57)).

#include <atomic>

#include "vmi_device.h"
#include "vmi_internal.h"

VMI_TL_DECL

namespace {

#pragma clang fp contract(off)

constexpr int kMaxK = 15;
constexpr int kBins = 2048;          // radix levels 1 and 2 (11 bits), level 3 uses 1024 (10 bits)
constexpr uint32_t kCtrTag = 0x5A3D1E57u;

__device__ __forceinline__ int acc_wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Degree-6 Taylor polynomial of 2^f, f in [-1/2, 1/2]: (ln 2)^k / k! in fp32.
__device__ __forceinline__ uint32_t sd_weight(float l, float M, float s2) {
    const float z = (l - M) * s2;
    if (!(z >= -32.0f)) return 0u;
    const float n = rintf(z);
    const float f = z - n;
    float p = 0x1.430912p-13f;
    p = __builtin_fmaf(p, f, 0x1.5d87fep-10f);
    p = __builtin_fmaf(p, f, 0x1.3b2ab6p-7f);
    p = __builtin_fmaf(p, f, 0x1.c6b08ep-5f);
    p = __builtin_fmaf(p, f, 0x1.ebfbep-3f);
    p = __builtin_fmaf(p, f, 0x1.62e43p-1f);
    p = __builtin_fmaf(p, f, 0x1p+0f);
    return (uint32_t)ldexpf(p, (int)n + 31);
}

__device__ __forceinline__ void philox(uint32_t c[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t hi0 = __umulhi(0xD2511F53u, c[0]), lo0 = 0xD2511F53u * c[0];
        const uint32_t hi1 = __umulhi(0xCD9E8D57u, c[2]), lo1 = 0xCD9E8D57u * c[2];
        const uint32_t n0 = hi1 ^ c[1] ^ k0;
        const uint32_t n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
}

__device__ __forceinline__ void sd_uniforms(uint64_t seed, uint64_t offset, int i, uint32_t& U, uint32_t& Vr) {
    uint32_t c[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), (uint32_t)i, kCtrTag};
    philox(c, (uint32_t)seed, (uint32_t)(seed >> 32));
    U = c[0];
    Vr = c[1];
}

constexpr int kSdThreads = 256;
constexpr int kSdWaves = kSdThreads / 64;
constexpr int kMaxRows = 64;         // distributions per call / rows per draw
constexpr int kHistAll = 2 * kBins + 1024;

struct SdStats {
    uint32_t theta;          // nucleus: W >= theta (theta >= 1)
    uint32_t valid;          // 0 when the row has no finite logit
    unsigned long long zs;   // nucleus mass
    unsigned long long z;    // total mass
    unsigned long long C;    // ceil(top_p * z)
    uint32_t b1, b2;
    unsigned long long above1, above2;
};

struct SdArgs {
    const float* base0;      // rows [0, n0)
    int n0;
    const float* base1;      // rows [n0, nd)
    int nd, V, NB, chunk;
    float s2, top_p;
    uint64_t seed, offset;   // the effective offset adds *offset_dev when that is set
    const uint64_t* offset_dev;
    uint32_t* status;        // caller's status word (VMI_STATUS_WAIT_GAVE_UP / BAD_LOGITS), or null
    int accept, K, has_q;    // accept mode: K drafts, draft rows present
    const int32_t* drafts;
    uint32_t* ctr_r;         // [kMaxRows] arrival counters of the draws
    SdStats* stats;          // [nd]
    float* pmax;             // [nd, NB]
    unsigned long long* hist;  // [nd, kHistAll]: level 1 | level 2 | level 3
    unsigned long long* partR; // [rows, NB]
    unsigned long long* partP; // [rows, NB]
    uint32_t* W;             // [nd, V]
    int32_t* out;            // accept: result record; sample: [rows]
};

__device__ __forceinline__ const float* sd_row(const SdArgs& a, int d) {
    return d < a.n0 ? a.base0 + (size_t)d * a.V : a.base1 + (size_t)(d - a.n0) * a.V;
}

// Adds v to bin b of an LDS histogram, merging runs of one bin per thread
// (most masses are tiny and share a bin: this keeps atomics off a hot spot).
struct BinRun {
    int bin = -1;
    unsigned long long sum = 0;
    __device__ void add(unsigned long long* h, int b, uint32_t v) {
        if (b != bin) {
            if (bin >= 0 && sum) atomicAdd(&h[bin], sum);
            bin = b;
            sum = 0;
        }
        sum += v;
    }
    __device__ void flush(unsigned long long* h) {
        if (bin >= 0 && sum) atomicAdd(&h[bin], sum);
        bin = -1;
        sum = 0;
    }
};

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int o) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, o);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), o);
    return ((uint64_t)hi << 32) | lo;
}

// Reverse inclusive scan over the lanes of a wave: lane l gets
// sum_{l' >= l} v(l').
__device__ __forceinline__ uint64_t suffix_scan64(uint64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, (lane + o) & 63);
        const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), (lane + o) & 63);
        if (lane + o < 64) v += ((uint64_t)hi << 32) | lo;
    }
    return v;
}

// Inclusive scan over the lanes of a wave: lane l gets sum_{l' <= l} v(l').
__device__ __forceinline__ uint64_t prefix_scan64(uint64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, (lane - o) & 63);
        const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), (lane - o) & 63);
        if (lane >= o) v += ((uint64_t)hi << 32) | lo;
    }
    return v;
}

// One wave: the largest bin b of h[0..nbins) with above + sum_{i >= b} h[i] >= C,
// and above + sum_{i > b} h[i].  Uniform results.  Lane l owns bins
// [l*per, (l+1)*per); the crossing lane comes from a suffix scan of the lane
// sums (the lanes meeting the target form a prefix, counted by a ballot),
// the crossing bin from a suffix scan of that lane's bins.
__device__ __forceinline__ void find_crossing(const unsigned long long* h, int nbins, uint64_t C, uint64_t above,
                                              uint32_t& b_out, uint64_t& above_out) {
    const int lane = threadIdx.x & 63;
    const int per = nbins / 64;
    uint64_t own = 0;
    for (int i = 0; i < per; ++i) own += h[lane * per + ((i + lane) & (per - 1))];  // rotated: no bank conflicts
    const uint64_t S = suffix_scan64(own);  // mass of lanes >= lane
    const int nl = __popcll(__ballot(above + S >= C));
    const int L = nl > 0 ? nl - 1 : 0;
    const uint64_t SL1 = L + 1 < 64 ? readlane64(S, L + 1) : 0ull;
    const uint64_t acc = above + (nl > 0 ? SL1 : readlane64(S, 0));
    // the bins of lane L, one per lane
    const uint64_t hv = lane < per ? h[L * per + lane] : 0ull;
    const uint64_t Tb = suffix_scan64(hv);  // mass of bins >= L*per + lane within lane L
    const int nb = __popcll(__ballot(lane < per && acc + Tb >= C));
    const int i = nb > 0 ? nb - 1 : 0;
    b_out = (uint32_t)(L * per + i);
    above_out = acc + (i + 1 < 64 ? readlane64(Tb, i + 1) : 0ull);
}

__device__ __forceinline__ uint64_t block_sum_u64(unsigned long long* red, uint64_t v) {
    const int lane = threadIdx.x & 63, w = acc_wave_id();
    for (int o = 32; o >= 1; o >>= 1) v += shfl_xor64(v, o);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    uint64_t t = 0;
    for (int i = 0; i < kSdWaves; ++i) t += red[i];
    __syncthreads();
    return t;
}

// Adds the non-zero bins of an LDS histogram into a global one.
__device__ __forceinline__ void flush_hist(const unsigned long long* lds, unsigned long long* g, int nbins) {
    for (int i = threadIdx.x; i < nbins; i += kSdThreads)
        if (lds[i]) atomicAdd(&g[i], lds[i]);
}

__device__ __forceinline__ void slice_of(const SdArgs& a, int b, int& j0, int& j1) {
    j0 = b * a.chunk;
    j1 = min(a.V, j0 + a.chunk);
}

// f(j, src[j]) for every j of [j0, j1) owned by this thread (stride
// kSdThreads), with kBatch loads in flight before any is used.
constexpr int kBatch = 8;
template <typename T, typename F>
__device__ __forceinline__ void for_slice(int j0, int j1, const T* __restrict__ src, F f) {
    for (int base = j0 + (int)threadIdx.x; base < j1; base += kBatch * kSdThreads) {
        T v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int j = base + u * kSdThreads;
            v[u] = j < j1 ? src[j] : T(0);
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int j = base + u * kSdThreads;
            if (j < j1) f(j, v[u]);
        }
    }
}

// One launch for the whole acceptance (or sampling) call: workgroup (b, d)
// owns slice b of distribution d through five phases, and all NB * nd
// workgroups are resident at once (the host sizes NB for that), so the
// phases meet at per-distribution arrival counters with bounded waits:
//   1. slice maxima; the distribution's histograms cleared
//   2. integer masses W of the slice (from the distribution's maximum),
//      level-1 histogram
//   3. the level-1 crossing bin (every workgroup of the distribution finds the
//      same one), level-2 histogram inside it
//   4. the level-2 crossing, level-3 histogram
//   5. workgroup 0 of the distribution fixes the nucleus threshold and mass
//      from the level-3 histogram and publishes them; the draw workgroups
//      wait until every distribution has, then run the draw (acceptance
//      decisions recomputed identically by every slice, masses of the
//      distribution to draw from per slice; the last slice of a draw to
//      finish finds the token).
// Every value that crosses workgroups (maxima, histograms, masses, the
// nucleus statistics, draw partial sums) is written and read with
// agent-scope (coherent) accesses, and a workgroup's stores have completed
// before it counts itself, so no fence writes back or invalidates the L2.
// Histograms are integer sums, so their value does not depend on arrival
// order, and the results equal those of the phases run as separate launches.
constexpr int kSdSpinLimit = 1 << 16;  // polls (each a coherent load) before a wait gives up, by default

struct SdSync {
    uint32_t* row;     // [kMaxRows] arrivals per distribution, 64 bytes apart (16 words)
    uint32_t* ready;   // distributions whose nucleus statistics are published
    uint32_t* done;    // distributions whose workgroups have all finished (the last resets every counter)
    uint32_t* rdone;   // [kMaxRows] workgroups of each distribution finished, 64 bytes apart
    uint32_t* flag;    // a wait gave up
    uint32_t* go;      // [nd * NB] per-workgroup release words, 64 bytes apart: the phase the workgroup may enter
    int spin_limit;    // polls before a wait gives up (>= 1)
};

__device__ __forceinline__ void sd_wait(uint32_t* c, uint32_t target, uint32_t* flag, int limit) {
    if (threadIdx.x == 0) {
        int spins = 0;
        while (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins >= limit) {
                __hip_atomic_fetch_or(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Phase barrier of the n workgroups sharing counter c: this workgroup's
// stores are complete, then it counts itself; the last to arrive (the counter
// at target - 1) raises the release word of each of the n workgroups to
// `phase`, and every workgroup waits on its own word (its own 64-byte line, so
// the waits do not all poll one address).
__device__ __forceinline__ void sd_barrier(uint32_t* c, uint32_t target, uint32_t* go, int n, int self,
                                           uint32_t phase, uint32_t* flag, int limit) {
    __shared__ int s_rel;
    vmi_vm_wait_c<0>();
    __syncthreads();
    if (threadIdx.x == 0)
        s_rel = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == target - 1u;
    __syncthreads();
    if (s_rel)
        for (int i = threadIdx.x; i < n; i += kSdThreads)
            __hip_atomic_store(go + 16 * i, phase, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sd_wait(go + 16 * self, phase, flag, limit);
}

__device__ __forceinline__ uint64_t ld64c(const unsigned long long* p) {
    return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64c(unsigned long long* p, uint64_t v) {
    __hip_atomic_store(p, (unsigned long long)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld32c(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Histogram bins [0, n) of g (written by other workgroups' atomics) into LDS,
// every load issued before any is used; returns the sum of this thread's bins.
template <int N>
__device__ __forceinline__ uint64_t hist_to_lds(const unsigned long long* g, unsigned long long* lds) {
    constexpr int PER = N / kSdThreads;
    const __amdgpu_buffer_rsrc_t rg = vmi_rsrc(g, (uint32_t)N * 8u);
    uint2 v[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) v[u] = vmi_bload_b64_coh(rg, (uint32_t)(threadIdx.x + kSdThreads * u) * 8u, 0);
    uint64_t sum = 0;
#pragma unroll
    for (int u = 0; u < PER; ++u) {
        const uint64_t x = ((uint64_t)v[u].y << 32) | v[u].x;
        lds[threadIdx.x + kSdThreads * u] = x;
        sum += x;
    }
    return sum;
}

// The nucleus statistics of distribution d as the draw reads them.
__device__ __forceinline__ SdStats sd_stats(const SdArgs& a, int d) {
    const SdStats* sp = &a.stats[d];
    SdStats s{};
    s.theta = ld32c(&sp->theta);
    s.valid = ld32c(&sp->valid);
    s.zs = ld64c(&sp->zs);
    return s;
}

__device__ __forceinline__ uint32_t nucleus_mass(const uint32_t* __restrict__ W, uint32_t theta, int j) {
    const uint32_t x = ld32c(W + j);
    return x >= theta ? x : 0u;
}

// What one draw samples from, recomputed identically by every workgroup.
struct DrawPlan {
    int bad;        // some distribution has no finite logit
    int m;          // accept mode: drafts kept
    int dp, dq;     // distribution rows of p (and q when residual with draft rows)
    int resid;      // residual max(0, p - q) instead of p
    int dm;         // draft token at the rejected position (one-hot q)
    uint32_t Vr;    // resampling uniform
    uint32_t th_p, th_q;
    double zp, zq;
};

__device__ __forceinline__ DrawPlan plan_draw(const SdArgs& a, int r) {
    DrawPlan P{};
    if (!a.accept) {
        const SdStats s = sd_stats(a, r);
        P.bad = !s.valid;
        P.dp = r;
        P.th_p = s.theta;
        P.zp = (double)s.zs;
        uint32_t U;
        sd_uniforms(a.seed, a.offset, r, U, P.Vr);
        return P;
    }
    // lane i loads what decision i needs (the statistics of p row i and q row
    // K + 1 + i and draft i's masses in both) and lane d the validity of
    // distribution d, all in one round of loads; the decisions are the
    // sequential rule's (the first rejected draft ends the run)
    const int lane = threadIdx.x & 63;
    const int K = a.K, V = a.V;
    P.bad = __ballot(lane < a.nd && !ld32c(&a.stats[lane < a.nd ? lane : 0].valid)) != 0ull;
    if (P.bad) return P;
    uint32_t thp = 0u, thq = 0u, wp = 0u, wq = 0u;
    uint64_t zp = 1ull, zq = 1ull;
    int dj = -1;
    if (lane <= K) {
        const SdStats sp = sd_stats(a, lane);
        thp = sp.theta;
        zp = sp.zs;
        if (lane < K) {
            dj = a.drafts[lane];
            if (a.has_q) {
                const SdStats sq = sd_stats(a, K + 1 + lane);
                thq = sq.theta;
                zq = sq.zs;
            }
            if (dj >= 0 && dj < V) {
                wp = ld32c(a.W + (size_t)lane * V + dj);
                if (a.has_q) wq = ld32c(a.W + (size_t)(K + 1 + lane) * V + dj);
            }
        }
    }
    bool keep = false;
    if (lane < K) {
        uint32_t U, Vr;
        sd_uniforms(a.seed, a.offset, lane, U, Vr);
        double pp = 0.0, qq = 1.0;
        if (dj >= 0 && dj < V) {
            pp = (double)(wp >= thp ? wp : 0u) / (double)zp;
            if (a.has_q) qq = (double)(wq >= thq ? wq : 0u) / (double)zq;
        }
        const double u = (double)U * 0x1p-32;
        keep = pp > 0.0 && u * qq <= pp;
    }
    const uint64_t rejected = __ballot(lane < K && !keep);
    const int m = rejected ? (int)__builtin_ctzll(rejected) : K;
    P.m = m;
    uint32_t U;
    sd_uniforms(a.seed, a.offset, m, U, P.Vr);
    P.dp = m;
    P.th_p = (uint32_t)__builtin_amdgcn_readlane((int)thp, m);
    P.zp = (double)readlane64(zp, m);
    P.resid = m < K;
    if (P.resid) {
        P.dm = __builtin_amdgcn_readlane(dj, m);
        if (a.has_q) {
            P.dq = K + 1 + m;
            P.th_q = (uint32_t)__builtin_amdgcn_readlane((int)thq, m);
            P.zq = (double)readlane64(zq, m);
        }
    }
    return P;
}

// floor(2^31 max(0, p(j) - q(j))) from the nucleus mass pm of p at j and the
// raw draft mass wq at j.
__device__ __forceinline__ uint32_t resid_value(const SdArgs& a, const DrawPlan& P, int j, uint32_t pm, uint32_t wq) {
    const double pj = (double)pm / P.zp;
    const double qj = a.has_q ? (double)(wq >= P.th_q ? wq : 0u) / P.zq : (j == P.dm ? 1.0 : 0.0);
    const double rr = pj - qj;
    return rr > 0.0 ? (uint32_t)(rr * 0x1p31) : 0u;
}

// The draw of row r by slice b; the last slice of the row to finish finds the
// token and writes the result.
__device__ __forceinline__ void sd_draw(const SdArgs& a, const SdSync& y, int r, int b, unsigned long long* s_scan,
                        unsigned long long* s_red) {
    __shared__ int s_last, s_bstar, s_tok;
    __shared__ unsigned long long s_base, s_t;
    __shared__ int s_use_p;
    const int tid = threadIdx.x, lane = tid & 63;
    const DrawPlan P = plan_draw(a, r);
    int j0, j1;
    slice_of(a, b, j0, j1);
    uint64_t sr = 0, sp = 0;
    if (!P.bad) {
        const __amdgpu_buffer_rsrc_t rp = vmi_rsrc(a.W + (size_t)P.dp * a.V, (uint32_t)a.V * 4u);
        const __amdgpu_buffer_rsrc_t rq =
            vmi_rsrc(a.W + (size_t)(a.has_q && P.resid ? P.dq : P.dp) * a.V, (uint32_t)a.V * 4u);
        for (int base = j0 + tid; base < j1; base += kBatch * kSdThreads) {
            uint32_t vp[kBatch], vq[kBatch];
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int j = base + u * kSdThreads;
                vp[u] = vmi_bload_b32_coh(rp, j < j1 ? (uint32_t)j * 4u : VMI_OOB, 0);
                vq[u] = vmi_bload_b32_coh(rq, j < j1 ? (uint32_t)j * 4u : VMI_OOB, 0);
            }
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                const int j = base + u * kSdThreads;
                if (j < j1) {
                    const uint32_t p = vp[u] >= P.th_p ? vp[u] : 0u;
                    sp += p;
                    if (P.resid) sr += resid_value(a, P, j, p, vq[u]);
                }
            }
        }
    }
    sr = block_sum_u64(s_red, sr);
    sp = block_sum_u64(s_red, sp);
    if (tid == 0) {
        st64c(&a.partR[r * a.NB + b], sr);
        st64c(&a.partP[r * a.NB + b], sp);
    }
    vmi_vm_wait_c<0>();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(&a.ctr_r[r], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (uint32_t)(a.NB - 1);
        if (s_last) __hip_atomic_store(&a.ctr_r[r], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!s_last) return;
    VMI_STAMP(r, 12);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (P.bad || ld32c(y.flag)) {
        if (tid == 0) {
            if (a.status)
                atomicOr(a.status, (P.bad ? VMI_STATUS_BAD_LOGITS : 0u) | (ld32c(y.flag) ? VMI_STATUS_WAIT_GAVE_UP : 0u));
            if (a.accept) {
                a.out[0] = 0; a.out[1] = 0; a.out[2] = 0; a.out[3] = -1;
            } else {
                a.out[r] = -1;
            }
        }
        return;
    }
    // totals, the slice holding the draw point, and the mass before it (wave 0;
    // lane i holds slices i and i + 64, NB <= 128)
    if (acc_wave_id() == 0) {
        const __amdgpu_buffer_rsrc_t rr = vmi_rsrc(a.partR + r * a.NB, (uint32_t)a.NB * 8u);
        const __amdgpu_buffer_rsrc_t rpp = vmi_rsrc(a.partP + r * a.NB, (uint32_t)a.NB * 8u);
        const uint2 r0v = vmi_bload_b64_coh(rr, (uint32_t)lane * 8u, 0), p0v = vmi_bload_b64_coh(rpp, (uint32_t)lane * 8u, 0);
        const uint2 r1v = vmi_bload_b64_coh(rr, (uint32_t)(lane + 64) * 8u, 0);
        const uint2 p1v = vmi_bload_b64_coh(rpp, (uint32_t)(lane + 64) * 8u, 0);
        const uint64_t r0 = ((uint64_t)r0v.y << 32) | r0v.x, p0 = ((uint64_t)p0v.y << 32) | p0v.x;
        const uint64_t r1 = ((uint64_t)r1v.y << 32) | r1v.x, p1 = ((uint64_t)p1v.y << 32) | p1v.x;
        uint64_t totR = r0 + r1, totP = p0 + p1;
        for (int o = 32; o >= 1; o >>= 1) {
            totR += shfl_xor64(totR, o);
            totP += shfl_xor64(totP, o);
        }
        const int use_p = !(P.resid && totR > 0);
        const uint64_t tot = use_p ? totP : totR;
        const uint64_t v0 = use_p ? p0 : r0, v1 = use_p ? p1 : r1;
        const uint64_t t = __umul64hi(tot, (uint64_t)P.Vr << 32);
        // the first slice whose inclusive prefix passes t, and the mass before
        // it (slices past NB load as zero)
        const uint64_t c0 = prefix_scan64(v0);
        const uint64_t c1 = readlane64(c0, 63) + prefix_scan64(v1);
        const uint64_t h0 = __ballot(c0 > t), h1 = __ballot(c1 > t);
        int bstar = a.NB - 1;  // unreachable fallback: t < total
        uint64_t acc = 0;
        if (h0) {
            bstar = (int)__builtin_ctzll(h0);
            acc = readlane64(c0, bstar) - readlane64(v0, bstar);
        } else if (h1) {
            const int i = (int)__builtin_ctzll(h1);
            bstar = i + 64;
            acc = readlane64(c1, i) - readlane64(v1, i);
        }
        if (lane == 0) {
            s_bstar = bstar;
            s_base = acc;
            s_t = t;
            s_use_p = use_p;
            s_tok = -1;
        }
    }
    __syncthreads();
    VMI_STAMP(r, 13);
    // inside slice b*: thread i owns the contiguous group of kBatch indices
    // k0 + kBatch i ..; an exclusive scan of the group sums finds the group
    // holding the draw point, whose owner walks it.
    const int bs = s_bstar, use_p = s_use_p;
    const uint64_t t = s_t;
    int k0, k1;
    slice_of(a, bs, k0, k1);
    const __amdgpu_buffer_rsrc_t sp_ = vmi_rsrc(a.W + (size_t)P.dp * a.V, (uint32_t)a.V * 4u);
    const __amdgpu_buffer_rsrc_t sq_ = vmi_rsrc(a.W + (size_t)(a.has_q && P.resid ? P.dq : P.dp) * a.V, (uint32_t)a.V * 4u);
    for (int g0 = k0; g0 < k1; g0 += kBatch * kSdThreads) {
        const int gj = g0 + kBatch * tid;
        uint32_t v[kBatch], wq[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const uint32_t off = gj + u < k1 ? (uint32_t)(gj + u) * 4u : VMI_OOB;
            v[u] = vmi_bload_b32_coh(sp_, off, 0);
            wq[u] = vmi_bload_b32_coh(sq_, off, 0);
        }
        uint64_t gs = 0;
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int j = gj + u;
            const uint32_t pm = v[u] >= P.th_p ? v[u] : 0u;
            v[u] = j < k1 ? (use_p ? pm : resid_value(a, P, j, pm, wq[u])) : 0u;
            gs += v[u];
        }
        // inclusive scan of the group sums over the workgroup: per wave, then
        // the preceding waves' totals
        const uint64_t ws = prefix_scan64(gs);
        if ((tid & 63) == 63) s_scan[acc_wave_id()] = ws;
        __syncthreads();
        uint64_t before = 0;
        for (int i = 0; i < acc_wave_id(); ++i) before += s_scan[i];
        uint64_t wtot = 0;
        for (int i = 0; i < kSdWaves; ++i) wtot += s_scan[i];
        const uint64_t base = s_base;
        const uint64_t incl = base + before + ws;
        uint64_t run = incl - gs;
        if (gs > 0 && run <= t && incl > t) {
#pragma unroll
            for (int u = 0; u < kBatch; ++u) {
                run += v[u];
                if (run > t) { s_tok = gj + u; break; }
            }
        }
        __syncthreads();
        if (tid == 0) s_base = base + wtot;
        __syncthreads();
        if (s_tok >= 0) break;
    }
    VMI_STAMP(r, 14);
    if (tid == 0) {
        int tok = s_tok;
        if (tok < 0) tok = k1 - 1;  // unreachable: t < total
        if (a.accept) {
            const int m = P.m;
            a.out[0] = m + 1;
            a.out[1] = m;
            a.out[2] = m + 1;
            a.out[3] = 0;
            for (int j = 0; j < m; ++j) a.out[4 + j] = a.drafts[j];
            a.out[4 + m] = tok;
        } else {
            a.out[r] = tok;
        }
    }
}

__global__ __launch_bounds__(kSdThreads) void k_sd_fused(SdArgs a, SdSync y, int rows) {
    if (a.offset_dev) a.offset += *a.offset_dev;
    __shared__ unsigned long long s_h[kBins];
    __shared__ unsigned long long s_red[kSdWaves];
    __shared__ float s_redf[kSdWaves];
    __shared__ uint32_t s_b1, s_pre;
    __shared__ unsigned long long s_above1, s_above2, s_C;
    __shared__ int s_valid;
    const int d = blockIdx.y, b = blockIdx.x, tid = threadIdx.x;
    const int NB = a.NB;
    uint32_t* rc = y.row + 16 * d;
    unsigned long long* h = a.hist + (size_t)d * kHistAll;
    int j0, j1;
    slice_of(a, b, j0, j1);
    const float* __restrict__ row = sd_row(a, d);
    uint32_t* W = a.W + (size_t)d * a.V;
    VMI_STAMP(d, 0);

    // 1. slice maximum; this workgroup's share of the histograms cleared
    float m0 = -INFINITY;
    for_slice(j0, j1, row, [&](int, float l) { m0 = fmaxf(m0, l); });
    {
        float m = vmi_wave_max(m0);
        if ((tid & 63) == 0) s_redf[acc_wave_id()] = m;
        for (int i = b * kSdThreads + tid; i < kHistAll; i += NB * kSdThreads) st64c(&h[i], 0ull);
        __syncthreads();
        if (tid == 0) {
            for (int i = 1; i < kSdWaves; ++i) m = fmaxf(m, s_redf[i]);
            __hip_atomic_store(&a.pmax[d * NB + b], m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    VMI_STAMP(d, 1);
    sd_barrier(rc, (uint32_t)NB, y.go + 16 * NB * d, NB, b, 1u, y.flag, y.spin_limit);
    VMI_STAMP(d, 2);

    // 2. masses and the level-1 histogram
    {
        float m = -INFINITY;
        for (int i = tid; i < NB; i += kSdThreads)
            m = fmaxf(m, __hip_atomic_load(&a.pmax[d * NB + i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        m = vmi_wave_max(m);
        if ((tid & 63) == 0) s_redf[acc_wave_id()] = m;
        for (int i = tid; i < kBins; i += kSdThreads) s_h[i] = 0ull;
        __syncthreads();
        float M = s_redf[0];
        for (int i = 1; i < kSdWaves; ++i) M = fmaxf(M, s_redf[i]);
        BinRun run;
        const float s2 = a.s2;
        for_slice(j0, j1, row, [&](int j, float l) {
            const uint32_t x = sd_weight(l, M, s2);
            __hip_atomic_store(W + j, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            run.add(s_h, (int)(x >> 21), x);
        });
        run.flush(s_h);
        __syncthreads();
        flush_hist(s_h, h, kBins);
    }
    VMI_STAMP(d, 3);
    sd_barrier(rc, 2u * NB, y.go + 16 * NB * d, NB, b, 2u, y.flag, y.spin_limit);
    VMI_STAMP(d, 4);

    // 3. total mass, nucleus target, level-1 crossing; level-2 histogram
    {
        const uint64_t part = hist_to_lds<kBins>(h, s_h);
        const uint64_t Z = block_sum_u64(s_red, part);
        if (Z > 0 && acc_wave_id() == 0) {
            uint64_t C = (a.top_p >= 1.0f) ? Z : (uint64_t)ceil((double)a.top_p * (double)Z);
            if (C == 0) C = 1;
            uint32_t b1;
            uint64_t above1;
            find_crossing(s_h, kBins, C, 0, b1, above1);
            if (tid == 0) {
                s_b1 = b1;
                s_above1 = above1;
                s_C = C;
            }
        }
        if (tid == 0) s_valid = Z > 0;
        __syncthreads();
        for (int i = tid; i < kBins; i += kSdThreads) s_h[i] = 0ull;
        __syncthreads();
        if (s_valid) {
            const uint32_t b1 = s_b1;
            BinRun run;
            for_slice(j0, j1, W, [&](int, uint32_t x) {
                if ((x >> 21) == b1) run.add(s_h, (int)((x >> 10) & 0x7ffu), x);
            });
            run.flush(s_h);
            __syncthreads();
            flush_hist(s_h, h + kBins, kBins);
        }
    }
    VMI_STAMP(d, 5);
    sd_barrier(rc, 3u * NB, y.go + 16 * NB * d, NB, b, 3u, y.flag, y.spin_limit);
    VMI_STAMP(d, 6);

    // 4. level-2 crossing; level-3 histogram
    if (s_valid) {
        hist_to_lds<kBins>(h + kBins, s_h);
        __syncthreads();
        if (acc_wave_id() == 0) {
            uint32_t b2;
            uint64_t above2;
            find_crossing(s_h, kBins, s_C, s_above1, b2, above2);
            if (tid == 0) {
                s_pre = (s_b1 << 11) | b2;
                s_above2 = above2;
            }
        }
        __syncthreads();
        const uint32_t pre = s_pre;
        for (int i = tid; i < 1024; i += kSdThreads) s_h[i] = 0ull;
        __syncthreads();
        BinRun run;
        for_slice(j0, j1, W, [&](int, uint32_t x) {
            if ((x >> 10) == pre) run.add(s_h, (int)(x & 0x3ffu), x);
        });
        run.flush(s_h);
        __syncthreads();
        flush_hist(s_h, h + 2 * kBins, 1024);
    }
    VMI_STAMP(d, 7);
    sd_barrier(rc, 4u * NB, y.go + 16 * NB * d, NB, b, 4u, y.flag, y.spin_limit);
    VMI_STAMP(d, 8);

    // 5. the nucleus of distribution d (its workgroup 0), then the draws
    if (b == 0) {
        SdStats* st = &a.stats[d];
        if (s_valid) {
            hist_to_lds<1024>(h + 2 * kBins, s_h);
            __syncthreads();
            if (acc_wave_id() == 0) {
                uint32_t b3;
                uint64_t above3;
                find_crossing(s_h, 1024, s_C, s_above2, b3, above3);
                if (tid == 0) {
                    __hip_atomic_store(&st->theta, (s_pre << 10) | b3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    st64c(&st->zs, above3 + s_h[b3]);
                }
            }
        }
        if (tid == 0) __hip_atomic_store(&st->valid, (uint32_t)s_valid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        vmi_vm_wait_c<0>();
        __syncthreads();
        __shared__ int s_rel5;
        if (tid == 0)
            s_rel5 = __hip_atomic_fetch_add(y.ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (uint32_t)a.nd - 1u;
        __syncthreads();
        if (s_rel5)
            for (int i = tid; i < rows * NB; i += kSdThreads)
                __hip_atomic_store(y.go + 16 * i, 5u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    VMI_STAMP(d, 9);
    if (d < rows) {
        sd_wait(y.go + 16 * (NB * d + b), 5u, y.flag, y.spin_limit);
        VMI_STAMP(d, 10);
        sd_draw(a, y, d, b, s_h, s_red);
        VMI_STAMP(d, 11);
    }
    // the last workgroup of the last distribution to finish clears the
    // counters for the next call (two levels, so no counter sees more than NB
    // arrivals)
    __shared__ int s_fin;
    vmi_vm_wait_c<0>();
    __syncthreads();
    if (tid == 0) {
        int fin = 0;
        if (__hip_atomic_fetch_add(y.rdone + 16 * d, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            (uint32_t)NB - 1u)
            fin = __hip_atomic_fetch_add(y.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                  (uint32_t)a.nd - 1u;
        s_fin = fin;
    }
    __syncthreads();
    if (s_fin) {
        for (int i = tid; i < a.nd * NB; i += kSdThreads)
            __hip_atomic_store(y.go + 16 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int i = tid; i < a.nd; i += kSdThreads) {
            __hip_atomic_store(y.row + 16 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(y.rdone + 16 * i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tid == 0) {
            __hip_atomic_store(y.ready, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(y.flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(y.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// ------------------------------------------------------------------ greedy
struct GreedyArgs {
    const int32_t* drafts;  // [P, K]
    const int32_t* preds;   // [P, K + mode]
    int P, K, mode;
    int32_t* result;        // [4 + K + 1]
};

__global__ __launch_bounds__(64) void k_accept_greedy(GreedyArgs a) {
    const int lane = threadIdx.x;
    const int K = a.K, Kp = a.K + a.mode;
    // lane p: matched length of path p; key = matched desc, then lower path
    int best = -1, bestp = 0;
    for (int p0 = 0; p0 < a.P; p0 += 64) {
        const int p = p0 + lane;
        int m = -1;
        if (p < a.P) {
            m = 0;
            while (m < K && a.preds[(size_t)p * Kp + m] == a.drafts[(size_t)p * K + m]) ++m;
        }
        const uint32_t key = m < 0 ? 0u : ((uint32_t)(m + 1) << 16) | (uint32_t)(0xffff - p);
        const uint32_t top = vmi_wave_max_u32(key);
        const int tm = (int)(top >> 16) - 1, tp = 0xffff - (int)(top & 0xffff);
        if (tm > best) { best = tm; bestp = tp; }
    }
    if (lane == 0) {
        const int32_t* dr = a.drafts + (size_t)bestp * K;
        const int32_t* pr = a.preds + (size_t)bestp * Kp;
        const int m = best;
        int n = 0;
        for (int j = 0; j < m; ++j) a.result[4 + n++] = dr[j];
        int acc_len;
        if (a.mode == 0) {
            if (m < K) a.result[4 + n++] = pr[m];
            acc_len = m + 1 < K ? m + 1 : K;
        } else {
            a.result[4 + n++] = pr[m];
            acc_len = m + 1;
        }
        a.result[0] = n;
        a.result[1] = m;
        a.result[2] = acc_len;
        a.result[3] = bestp;
    }
}

// Workspace: counters first (fixed offsets whatever the shape, zero between
// calls): the per-distribution phase counters one 64-byte line each, the
// ready / done / gave-up words and the draws' counters; then per-row state.
constexpr int kSdMaxWgs = 2048;  // release words (one 64-byte line per workgroup of a launch)
constexpr size_t kSdSyncBytes = 64 * kMaxRows + 256 + kMaxRows * sizeof(uint32_t) + 64 * kSdMaxWgs + 64 * kMaxRows;

struct SdLayout {
    size_t stats, pmax, hist, partR, partP, W, bytes;
};

SdLayout sd_layout(int nd, int rows, int V, int NB) {
    SdLayout L{};
    size_t off = vmi::align256(kSdSyncBytes);
    L.stats = off; off += vmi::align256((size_t)nd * sizeof(SdStats));
    L.pmax = off; off += vmi::align256((size_t)nd * NB * sizeof(float));
    L.hist = off; off += vmi::align256((size_t)nd * kHistAll * sizeof(unsigned long long));
    L.partR = off; off += vmi::align256((size_t)rows * NB * sizeof(unsigned long long));
    L.partP = off; off += vmi::align256((size_t)rows * NB * sizeof(unsigned long long));
    L.W = off; off += vmi::align256((size_t)nd * V * sizeof(uint32_t));
    L.bytes = off;
    return L;
}

// Slices per row: at most kBatch * kSdThreads = 2048 logits each (one batch
// of loads per thread), at most 128 slices.
int sd_slices(int V) {
    int nb = (V + kBatch * kSdThreads - 1) / (kBatch * kSdThreads);
    return nb < 1 ? 1 : (nb > 128 ? 128 : nb);
}

// Workgroups of k_sd_fused one compute unit holds at once, from the
// occupancy calculator (registers, LDS), at most two: the waits need every
// workgroup of a launch resident, and a second one per CU leaves room for
// other work on the device.  Queried once per device (re-entrant as
// vmi::device_cus).
int sd_resident_per_cu() {
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    const int known = cached[dev].load(std::memory_order_relaxed);
    if (known > 0) return known;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k_sd_fused, kSdThreads, 0) != hipSuccess || n < 1) n = 1;
    if (n > 2) n = 2;
    cached[dev].store(n, std::memory_order_relaxed);
    return n;
}

// Bound of the kernel's co-residency waits (polls); vmi_set_wait_limit.
std::atomic<int> g_sd_spin_limit{kSdSpinLimit};

// Slices per row for a launch of nd distributions: every workgroup of the
// launch must be resident at once, so NB * nd <= sd_resident_per_cu() * CUs.
int sd_slices_resident(int V, int nd) {
    int cap = sd_resident_per_cu() * vmi::device_cus() / nd;
    if (cap * nd > kSdMaxWgs) cap = kSdMaxWgs / nd;
    const int nb = sd_slices(V);
    return nb < cap ? nb : (cap < 1 ? 1 : cap);
}

float sd_scale(float temperature) { return (float)((1.0 / (double)temperature) * 1.4426950408889634); }

hipError_t sd_launch(SdArgs& a, uint8_t* ws, int rows, hipStream_t s) {
    SdSync y{};
    y.row = reinterpret_cast<uint32_t*>(ws);
    y.ready = reinterpret_cast<uint32_t*>(ws + 64 * kMaxRows);
    y.done = reinterpret_cast<uint32_t*>(ws + 64 * kMaxRows + 64);
    y.flag = reinterpret_cast<uint32_t*>(ws + 64 * kMaxRows + 128);
    a.ctr_r = reinterpret_cast<uint32_t*>(ws + 64 * kMaxRows + 256);
    y.go = reinterpret_cast<uint32_t*>(ws + 64 * kMaxRows + 256 + kMaxRows * sizeof(uint32_t));
    y.rdone = reinterpret_cast<uint32_t*>(ws + 64 * kMaxRows + 256 + kMaxRows * sizeof(uint32_t) + 64 * kSdMaxWgs);
    y.spin_limit = g_sd_spin_limit.load(std::memory_order_relaxed);
    hipLaunchKernelGGL(k_sd_fused, dim3(a.NB, a.nd), dim3(kSdThreads), 0, s, a, y, rows);
    return hipGetLastError();
}

void sd_bind(SdArgs& a, uint8_t* ws, const SdLayout& L) {
    a.stats = reinterpret_cast<SdStats*>(ws + L.stats);
    a.pmax = reinterpret_cast<float*>(ws + L.pmax);
    a.hist = reinterpret_cast<unsigned long long*>(ws + L.hist);
    a.partR = reinterpret_cast<unsigned long long*>(ws + L.partR);
    a.partP = reinterpret_cast<unsigned long long*>(ws + L.partP);
    a.W = reinterpret_cast<uint32_t*>(ws + L.W);
}

// The commit of one speculative step from k_accept_greedy's record, in either
// verify layout: with acc = accepted_len and w = the winning path,
// H = hid[w][acc - 1], x = the last emitted token, pos += acc,
// mtp_len += acc and the next step's draft positions mtp_len + i.  A record
// outside what the call allows (no emitted token, acc outside [1, rows], more
// than rows + 1 tokens, a path outside [0, paths)) changes nothing and sets
// VMI_STATUS_BAD_RECORD.  One workgroup: the threads copy the hidden row,
// thread 0 the scalars.
struct CommitArgs {
    const int32_t* rec;
    const uint16_t* hid;
    int rows, paths, hidden, K;
    uint16_t* H;
    int32_t* x;
    int32_t* pos;
    int32_t* mtp_len;
    int32_t* mtp_pos;
    uint32_t* status;
};

__global__ __launch_bounds__(256) void k_spec_commit(CommitArgs a) {
    const int n = a.rec[0], acc = a.rec[2], w = a.rec[3];
    // a valid record emits at most one token per verify row
    if (n < 1 || n > a.rows || acc < 1 || acc > a.rows || w < 0 || w >= a.paths) {
        if (threadIdx.x == 0 && a.status) atomicOr(a.status, VMI_STATUS_BAD_RECORD);
        return;
    }
    const uint16_t* src = a.hid + ((size_t)w * a.rows + acc - 1) * a.hidden;
    for (int i = threadIdx.x; i < a.hidden; i += 256) a.H[i] = src[i];
    if (threadIdx.x == 0) {
        a.x[0] = a.rec[4 + n - 1];
        a.pos[0] += acc;
        const int ml = a.mtp_len[0] + acc;
        a.mtp_len[0] = ml;
        for (int i = 0; i < a.K; ++i) a.mtp_pos[i] = ml + i;
    }
}

}  // namespace

extern "C" int vmi_accept_greedy(const int32_t* drafts, const int32_t* preds, int P, int K, int mode, int32_t* result,
                                 void* stream) {
    vmi::clear_error();
    if (P <= 0 || P > 0xffff || K <= 0 || K > kMaxK) return vmi::fail(VMI_ERR_INVALID, "P=%d K=%d", P, K);
    if (mode != 0 && mode != 1) return vmi::fail(VMI_ERR_INVALID, "mode=%d", mode);
    if (mode == 1 && P != 1) return vmi::fail(VMI_ERR_INVALID, "mode 1 (K+1 verify rows) takes one chain");
    if (!drafts || !preds || !result) return vmi::fail(VMI_ERR_INVALID, "null drafts/preds/result");
    GreedyArgs g{drafts, preds, P, K, mode, result};
    hipLaunchKernelGGL(k_accept_greedy, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), g);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_accept_greedy launch");
}

extern "C" int vmi_spec_commit(const int32_t* result, const uint16_t* hid, int rows, int paths, int hidden, int K,
                               uint16_t* H, int32_t* x, int32_t* pos, int32_t* mtp_len, int32_t* mtp_pos,
                               uint32_t* status, void* stream) {
    vmi::clear_error();
    if (K <= 0 || K > kMaxK || hidden <= 0) return vmi::fail(VMI_ERR_INVALID, "K=%d hidden=%d", K, hidden);
    if (rows <= 0 || rows > kMaxK + 1 || paths <= 0 || paths > 0xffff)
        return vmi::fail(VMI_ERR_INVALID, "rows=%d paths=%d", rows, paths);
    if (!result || !hid || !H || !x || !pos || !mtp_len || !mtp_pos)
        return vmi::fail(VMI_ERR_INVALID, "null result/hid/H/x/pos/mtp_len/mtp_pos");
    const uintptr_t hb = reinterpret_cast<uintptr_t>(hid), he = hb + (size_t)paths * rows * hidden * 2;
    const uintptr_t Hb = reinterpret_cast<uintptr_t>(H), Hend = Hb + (size_t)hidden * 2;
    if (Hb < he && hb < Hend) return vmi::fail(VMI_ERR_INVALID, "H overlaps hid");
    CommitArgs c{result, hid, rows, paths, hidden, K, H, x, pos, mtp_len, mtp_pos, status};
    hipLaunchKernelGGL(k_spec_commit, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), c);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "k_spec_commit launch");
}

extern "C" size_t vmi_accept_stochastic_workspace_bytes(int K, int vocab, int has_draft_logits) {
    if (K <= 0 || K > kMaxK || vocab <= 0) return 0;
    const int nd = (K + 1) + (has_draft_logits ? K : 0);
    return sd_layout(nd, 1, vocab, sd_slices(vocab)).bytes;
}

extern "C" int vmi_accept_stochastic(const float* target_logits, const float* draft_logits, const int32_t* drafts,
                                     int K, int vocab, float temperature, float top_p, uint64_t seed, uint64_t offset,
                                     const uint64_t* offset_device, int32_t* result, void* workspace,
                                     size_t workspace_bytes, uint32_t* status, void* stream) {
    vmi::clear_error();
    if (K <= 0 || K > kMaxK) return vmi::fail(VMI_ERR_UNSUPPORTED, "K=%d must be in [1, %d]", K, kMaxK);
    if (vocab <= 0 || vocab > (1 << 24)) return vmi::fail(VMI_ERR_INVALID, "vocab=%d", vocab);
    if (!(temperature > 0.0f) || !(temperature < 1e30f))
        return vmi::fail(VMI_ERR_INVALID, "temperature must be positive (use vmi_accept_greedy for 0)");
    if (!(top_p > 0.0f) || top_p > 1.0f) return vmi::fail(VMI_ERR_INVALID, "top_p must be in (0, 1]");
    if (!target_logits || !drafts || !result) return vmi::fail(VMI_ERR_INVALID, "null target/drafts/result");
    const int nd = (K + 1) + (draft_logits ? K : 0);
    const SdLayout L = sd_layout(nd, 1, vocab, sd_slices(vocab));
    const int NB = sd_slices_resident(vocab, nd);
    if (!workspace || workspace_bytes < L.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", L.bytes, workspace_bytes);
    SdArgs a{};
    a.base0 = target_logits; a.n0 = K + 1; a.base1 = draft_logits;
    a.nd = nd; a.V = vocab; a.NB = NB; a.chunk = (vocab + NB - 1) / NB;
    a.s2 = sd_scale(temperature); a.top_p = top_p; a.seed = seed; a.offset = offset;
    a.offset_dev = offset_device; a.status = status;
    a.accept = 1; a.K = K; a.has_q = draft_logits != nullptr; a.drafts = drafts;
    a.out = result;
    sd_bind(a, static_cast<uint8_t*>(workspace), L);
    const hipError_t e = sd_launch(a, static_cast<uint8_t*>(workspace), 1, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "stochastic acceptance launch");
}

extern "C" size_t vmi_sample_top_p_workspace_bytes(int rows, int vocab) {
    if (rows <= 0 || rows > kMaxRows || vocab <= 0) return 0;
    return sd_layout(rows, rows, vocab, sd_slices(vocab)).bytes;
}

extern "C" int vmi_sample_top_p(const float* logits, int rows, int vocab, float temperature, float top_p,
                                uint64_t seed, uint64_t offset, const uint64_t* offset_device, int32_t* out,
                                void* workspace, size_t workspace_bytes, uint32_t* status, void* stream) {
    vmi::clear_error();
    if (rows <= 0 || rows > kMaxRows) return vmi::fail(VMI_ERR_UNSUPPORTED, "rows=%d must be in [1, %d]", rows, kMaxRows);
    if (vocab <= 0 || vocab > (1 << 24)) return vmi::fail(VMI_ERR_INVALID, "vocab=%d", vocab);
    if (!(temperature > 0.0f) || !(temperature < 1e30f)) return vmi::fail(VMI_ERR_INVALID, "temperature must be positive");
    if (!(top_p > 0.0f) || top_p > 1.0f) return vmi::fail(VMI_ERR_INVALID, "top_p must be in (0, 1]");
    if (!logits || !out) return vmi::fail(VMI_ERR_INVALID, "null logits/out");
    const SdLayout L = sd_layout(rows, rows, vocab, sd_slices(vocab));
    const int NB = sd_slices_resident(vocab, rows);
    if (!workspace || workspace_bytes < L.bytes)
        return vmi::fail(VMI_ERR_WORKSPACE, "workspace needs %zu bytes (got %zu)", L.bytes, workspace_bytes);
    SdArgs a{};
    a.base0 = logits; a.n0 = rows; a.base1 = nullptr;
    a.nd = rows; a.V = vocab; a.NB = NB; a.chunk = (vocab + NB - 1) / NB;
    a.s2 = sd_scale(temperature); a.top_p = top_p; a.seed = seed; a.offset = offset;
    a.offset_dev = offset_device; a.status = status;
    a.accept = 0; a.K = 0; a.has_q = 0; a.drafts = nullptr;
    a.out = out;
    sd_bind(a, static_cast<uint8_t*>(workspace), L);
    const hipError_t e = sd_launch(a, static_cast<uint8_t*>(workspace), rows, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? VMI_OK : vmi::hip_fail(e, "top-p sampling launch");
}

#ifdef VMI_TIMELINE
// Tuning builds only: where the kernels of this file record their stamps.
extern "C" int vmi_timeline_set_accept(void* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(vmi_tl_buf), &buf, sizeof(buf)) == hipSuccess ? VMI_OK : VMI_ERR_HIP;
}
#endif

extern "C" int vmi_set_wait_limit(int polls) {
    const int prev = g_sd_spin_limit.load(std::memory_order_relaxed);
    g_sd_spin_limit.store(polls > 0 ? polls : kSdSpinLimit, std::memory_order_relaxed);
    return prev;
}
