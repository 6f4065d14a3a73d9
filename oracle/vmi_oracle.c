/*
 * vmi_oracle.c -- CPU oracle for the speculative-decode MoE hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or as the reported CPU baseline.  The product path (vates_amd) never calls it.
 *
 * Every function restates the reference algorithm it cites (paths are relative
 * to the AMOS144/Vates checkout).  Floating-point "truth" paths accumulate in
 * double; the router path reproduces the GPU kernel's fp32 operation order
 * exactly so that routed expert ids are bit-identical.  Build with
 * -ffp-contract=off: every fused multiply-add below is written as fmaf().
 *
 * Pinning (see tests/test_oracle_*.py):
 *   philox          Random123 known-answer vectors
 *   dequant         closed-form nibble order / affine values; reference fixture
 *                   (test_native_moe_ext.py:20-47 weight=arange, scale=bf16(0.001))
 *   quantize        round-trip bound |w - deq| <= s/2 (+ bf16 edge), brute force
 *   qgemv / experts numpy float64 matmul of the dequantised matrices
 *   route/top-k     numpy argsort brute force, tie rule, scipy softmax
 *   route reduce    literal known answer test_expert_major_prefill.py:89-103
 *   expert-major    literal known answer test_expert_major_prefill.py:33-60
 *   accept greedy   literal known answers test_mtp_generate.py:211-223,
 *                   spec == non-spec greedy invariant on toy models
 *   accept stoch.   exact output-distribution enumeration on tiny vocabularies
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>
#include <omp.h>

#define ORC_OK 0
#define ORC_EINVAL -1
#define ORC_ESLOT -2
#define ORC_ENOMEM -3

/* ------------------------------------------------------------------ bf16 */
static inline float bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even fp32 -> bf16 (NaN kept quiet). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t v) { return bf16_to_f32(v); }

/* ---------------------------------------------------------------- Philox */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As
 * Easy as 1, 2, 3", SC'11).  Integer-only, so the GPU generator produces the
 * same words. */
void orc_philox4x32_10(const uint32_t ctr_in[4], const uint32_t key_in[2], uint32_t out[4]) {
    uint32_t c0 = ctr_in[0], c1 = ctr_in[1], c2 = ctr_in[2], c3 = ctr_in[3];
    uint32_t k0 = key_in[0], k1 = key_in[1];
    for (int r = 0; r < 10; ++r) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* Irwin-Hall(4) approximate normal: element i of stream `stream` under `seed`
 * is ((u0+u1+u2+u3) - 131070) * scale with u* the four 16-bit halves of one
 * Philox half-block.  `scale` = std / 37837.2265 (the Irwin-Hall std of four
 * uniform 16-bit words).  The integer sum and one fp32 multiply are exact
 * across CPU and GPU, so synthetic tensors are bit-identical. */
static inline float synth_one(uint64_t seed, uint32_t stream, uint64_t i, float scale) {
    uint32_t ctr[4] = {(uint32_t)(i >> 1), (uint32_t)(i >> 33), stream, 0x5eed0001u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    orc_philox4x32_10(ctr, key, o);
    uint32_t a = (i & 1) ? o[2] : o[0];
    uint32_t b = (i & 1) ? o[3] : o[1];
    int32_t s = (int32_t)((a & 0xffffu) + (a >> 16) + (b & 0xffffu) + (b >> 16)) - 131070;
    return (float)s * scale;
}

void orc_synth_normal(uint64_t seed, uint32_t stream, uint64_t n, float scale, float* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = synth_one(seed, stream, i, scale);
}

void orc_synth_normal_bf16(uint64_t seed, uint32_t stream, uint64_t n, float scale, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(synth_one(seed, stream, i, scale));
}

/* ------------------------------------------------------------ quantise */
/* Affine quantiser used to make fixture and synthetic weights.  It follows the
 * reference's own CPU restatement native/bench/compute/qlinear_bench.cpp:37-80
 * (per-group min/max, scale=(max-min)/qmax, bias=min, round, clamp, LSB-first
 * packing), with one documented change: scale and bias are rounded to bf16
 * first and q is computed against the rounded values, as the packed format
 * stores bf16 scales/biases (native_moe.py:57-72).
 * Packing: value at column c occupies bits (c*bits)%32 of word (c*bits)/32
 * of its row (fused_moe.cpp:131-145).  bits in {4, 8}. */
static void quant_row(const float* w, int cols, int group, int bits, uint32_t* wq, uint16_t* s, uint16_t* b) {
    int groups = cols / group;
    int words = cols * bits / 32;
    int qmax = (1 << bits) - 1;
    memset(wq, 0, sizeof(uint32_t) * (size_t)words);
    for (int g = 0; g < groups; ++g) {
        const float* v = w + (size_t)g * group;
        float mn = v[0], mx = v[0];
        for (int i = 1; i < group; ++i) {
            if (v[i] < mn) mn = v[i];
            if (v[i] > mx) mx = v[i];
        }
        float scale = (mx - mn) / (float)qmax;
        if (scale == 0.0f) scale = 1.0f;
        uint16_t sb = orc_f32_to_bf16(scale);
        uint16_t bb = orc_f32_to_bf16(mn);
        float sf = bf16_to_f32(sb), bf = bf16_to_f32(bb);
        if (sf == 0.0f) { sb = 0x3f80; sf = 1.0f; }
        s[g] = sb;
        b[g] = bb;
        for (int i = 0; i < group; ++i) {
            int c = g * group + i;
            float qf = roundf((v[i] - bf) / sf);
            int q = (int)qf;
            if (!(qf >= 0.0f)) q = 0;
            if (q > qmax) q = qmax;
            int bit = c * bits;
            wq[bit / 32] |= ((uint32_t)q) << (bit % 32);
        }
    }
}

int orc_quantize_affine(const float* w, int rows, int cols, int group, int bits,
                        uint32_t* wq, uint16_t* s, uint16_t* b) {
    if (rows <= 0 || cols <= 0 || group <= 0 || cols % group || (bits != 4 && bits != 8) || (cols * bits) % 32)
        return ORC_EINVAL;
    int words = cols * bits / 32, groups = cols / group;
    for (int r = 0; r < rows; ++r)
        quant_row(w + (size_t)r * cols, cols, group, bits, wq + (size_t)r * words, s + (size_t)r * groups,
                  b + (size_t)r * groups);
    return ORC_OK;
}

/* Synthetic N(0, std)-like matrix [rows, cols] drawn with orc_synth_normal
 * (element index r*cols+c) and quantised with orc_quantize_affine. */
int orc_synth_quantized(uint64_t seed, uint32_t stream, int rows, int cols, int group, int bits, float scale,
                        uint32_t* wq, uint16_t* s, uint16_t* b) {
    if (rows <= 0 || cols <= 0 || group <= 0 || cols % group || (bits != 4 && bits != 8) || (cols * bits) % 32)
        return ORC_EINVAL;
    float* row = (float*)malloc(sizeof(float) * (size_t)cols);
    if (!row) return ORC_ENOMEM;
    int words = cols * bits / 32, groups = cols / group;
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < cols; ++c) row[c] = synth_one(seed, stream, (uint64_t)r * cols + c, scale);
        quant_row(row, cols, group, bits, wq + (size_t)r * words, s + (size_t)r * groups, b + (size_t)r * groups);
    }
    free(row);
    return ORC_OK;
}

/* ------------------------------------------------------------- dequant */
/* qvalue (fused_moe.cpp:131-145; custom_kernel.py:170-184):
 *   q = (w[row, (c*bits)/32] >> ((c*bits)%32)) & (2^bits-1)
 *   w = q * scale[row, c/group] + bias[row, c/group]
 * q*scale is exact in fp32 (<= 8-bit q times an 8-bit bf16 significand), so the
 * single rounding of the add makes this value FMA-invariant. */
static inline float deq(const uint32_t* wrow, const uint16_t* srow, const uint16_t* brow, int c, int group, int bits) {
    int bit = c * bits;
    uint32_t q = wrow[bit / 32] >> (bit % 32);
    if ((bit % 32) + bits > 32) q |= wrow[bit / 32 + 1] << (32 - bit % 32);
    q &= (1u << bits) - 1u;
    int g = c / group;
    return fmaf((float)q, bf16_to_f32(srow[g]), bf16_to_f32(brow[g]));
}

int orc_dequant_affine(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int rows, int cols, int group,
                       int bits, float* out) {
    if (rows <= 0 || cols <= 0 || group <= 0 || cols % group || bits < 1 || bits > 8 || (cols * bits) % 32)
        return ORC_EINVAL;
    int words = cols * bits / 32, groups = cols / group;
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < cols; ++c)
            out[(size_t)r * cols + c] = deq(wq + (size_t)r * words, s + (size_t)r * groups, b + (size_t)r * groups, c,
                                            group, bits);
    return ORC_OK;
}

/* y[t, r] = sum_c deq(W)[r, c] * x[t, c], double accumulation. */
static void qgemv_f64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int rows, int cols, int group,
                      int bits, const double* x, int T, double* y) {
    int words = cols * bits / 32, groups = cols / group;
    for (int r = 0; r < rows; ++r) {
        const uint32_t* wr = wq + (size_t)r * words;
        const uint16_t* sr = s + (size_t)r * groups;
        const uint16_t* br = b + (size_t)r * groups;
        for (int t = 0; t < T; ++t) {
            double acc = 0.0;
            const double* xt = x + (size_t)t * cols;
            for (int c = 0; c < cols; ++c) acc += (double)deq(wr, sr, br, c, group, bits) * xt[c];
            y[(size_t)t * rows + r] = acc;
        }
    }
}

int orc_qgemv_f64(const uint32_t* wq, const uint16_t* s, const uint16_t* b, int rows, int cols, int group, int bits,
                  const float* x, int T, double* y) {
    if (rows <= 0 || cols <= 0 || T <= 0 || cols % group || (cols * bits) % 32) return ORC_EINVAL;
    double* xd = (double*)malloc(sizeof(double) * (size_t)T * cols);
    if (!xd) return ORC_ENOMEM;
    for (size_t i = 0; i < (size_t)T * cols; ++i) xd[i] = x[i];
    qgemv_f64(wq, s, b, rows, cols, group, bits, xd, T, y);
    free(xd);
    return ORC_OK;
}

/* Sum of 64 lane partials in the GPU's canonical wave-reduction tree
 * (vmi_wave_sum_canon): inside each 16-lane row a[l] + a[l^1], then + [l^2],
 * then + the lane mirrored inside its 8-lane half row, then + the lane
 * mirrored inside its 16-lane row; the four row sums as (R0 + R1) + (R2 + R3). */
static float canon_sum64(const float* a) {
    float b[64], c[64], d[64], e[64];
    for (int l = 0; l < 64; ++l) b[l] = a[l] + a[l ^ 1];
    for (int l = 0; l < 64; ++l) c[l] = b[l] + b[l ^ 2];
    for (int l = 0; l < 64; ++l) d[l] = c[l] + c[(l & ~7) | (7 - (l & 7))];
    for (int l = 0; l < 64; ++l) e[l] = d[l] + d[(l & ~15) | (15 - (l & 15))];
    return (e[0] + e[16]) + (e[32] + e[48]);
}

/* -------------------------------------------------------------- router */
/* Router logits in the GPU kernel's exact fp32 order (k_router in
 * vates_amd/csrc/vmi_moe.hip): lane l of a 64-lane wave owns columns
 * [l*cpl, (l+1)*cpl) with cpl = cols/64 and accumulates acc = fmaf(deq, x,
 * acc) in column order; the 64 partials meet in canon_sum64.  The logit bias,
 * if any, is added last.
 * Semantics: raw_gates = self.gate(x) (block.py:251-253). */
static float router_row_f32(const uint32_t* wr, const uint16_t* sr, const uint16_t* br, int cols, int group, int bits,
                            const float* xt) {
    float a[64];
    int cpl = cols / 64;
    for (int l = 0; l < 64; ++l) {
        float acc = 0.0f;
        for (int j = 0; j < cpl; ++j) {
            int c = l * cpl + j;
            acc = fmaf(deq(wr, sr, br, c, group, bits), xt[c], acc);
        }
        a[l] = acc;
    }
    return canon_sum64(a);
}

int orc_router_logits_f32(const uint32_t* wq, const uint16_t* s, const uint16_t* b, const float* logit_bias, int E,
                          int H, int group, int bits, const uint16_t* x_bf16, int T, float* logits) {
    if (E <= 0 || T <= 0 || H % 64 || H % group || (H / 64) % 8) return ORC_EINVAL;
    int words = H * bits / 32, groups = H / group;
    float* xt = (float*)malloc(sizeof(float) * (size_t)H);
    if (!xt) return ORC_ENOMEM;
    for (int t = 0; t < T; ++t) {
        for (int c = 0; c < H; ++c) xt[c] = bf16_to_f32(x_bf16[(size_t)t * H + c]);
        for (int e = 0; e < E; ++e) {
            float v = router_row_f32(wq + (size_t)e * words, s + (size_t)e * groups, b + (size_t)e * groups, H, group,
                                     bits, xt);
            if (logit_bias) v = v + logit_bias[e];
            logits[(size_t)t * E + e] = v;
        }
    }
    free(xt);
    return ORC_OK;
}

/* Top-k routing (block.py:321-329; qwen3_next_mtp.py:124-128):
 *   gates = softmax(raw, precise) ; inds = top-k(gates) ; s = gates[inds]
 *   if norm_topk_prob: s /= sum(s)
 * Selection is made on the logits (softmax is monotone), ordered by logit
 * descending, ties to the lower expert index (argpartition leaves ties
 * unspecified, block.py:323); NaN logits rank below every number.
 * Scores in double. */
static int better(float a, int ia, float b, int ib) {
    int na = isnan(a), nb = isnan(b);
    if (na != nb) return nb;
    if (!na && a != b) return a > b;
    return ia < ib;
}

int orc_topk_softmax(const float* logits, int T, int E, int k, int norm, int32_t* ids, float* scores) {
    if (T <= 0 || E <= 0 || k <= 0 || k > E || k > 64) return ORC_EINVAL;
    for (int t = 0; t < T; ++t) {
        const float* l = logits + (size_t)t * E;
        int sel[64];
        for (int j = 0; j < k; ++j) {
            int best = -1;
            for (int e = 0; e < E; ++e) {
                int used = 0;
                for (int q = 0; q < j; ++q) used |= (sel[q] == e);
                if (used) continue;
                if (best < 0 || better(l[e], e, l[best], best)) best = e;
            }
            sel[j] = best;
        }
        double m = -INFINITY;
        for (int e = 0; e < E; ++e)
            if (!isnan(l[e]) && l[e] > m) m = l[e];
        double denom = 0.0;
        if (norm) {
            for (int j = 0; j < k; ++j) denom += exp((double)l[sel[j]] - m);
        } else {
            for (int e = 0; e < E; ++e) denom += exp((double)l[e] - m);
        }
        for (int j = 0; j < k; ++j) {
            ids[(size_t)t * k + j] = sel[j];
            scores[(size_t)t * k + j] = (float)(exp((double)l[sel[j]] - m) / denom);
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------- experts */
typedef struct {
    const uint32_t *gw, *uw, *dw;
    const uint16_t *gs, *gb, *us, *ub, *ds, *db;
} orc_pool;

/* One SwiGLU expert on one token (fused_moe.cpp:221-283; custom_kernel.py:263-339):
 *   g = Wg x ; u = Wu x ; a = g * sigmoid(g) * u ; y = Wd a      (double) */
static void expert_f64(const orc_pool* p, int slot, const double* x, int H, int I, int group, int bits, double* a,
                       double* y) {
    size_t gu_words = (size_t)H * bits / 32, gu_groups = (size_t)H / group;
    size_t d_words = (size_t)I * bits / 32, d_groups = (size_t)I / group;
    for (int r = 0; r < I; ++r) {
        size_t row = (size_t)slot * I + r;
        double g = 0.0, u = 0.0;
        for (int c = 0; c < H; ++c) {
            g += (double)deq(p->gw + row * gu_words, p->gs + row * gu_groups, p->gb + row * gu_groups, c, group, bits) * x[c];
            u += (double)deq(p->uw + row * gu_words, p->us + row * gu_groups, p->ub + row * gu_groups, c, group, bits) * x[c];
        }
        a[r] = g * (1.0 / (1.0 + exp(-g))) * u;
    }
    for (int h = 0; h < H; ++h) {
        size_t row = (size_t)slot * H + h;
        double acc = 0.0;
        for (int r = 0; r < I; ++r)
            acc += (double)deq(p->dw + row * d_words, p->ds + row * d_groups, p->db + row * d_groups, r, group, bits) * a[r];
        y[h] = acc;
    }
}

/* fused_moe_slots (bindings.cpp:300-320; fused_moe.cpp:514-556, 635-664):
 * x f32 [T, H]; local_slots [T*k] token-major (token = pair / k,
 * fused_moe.cpp:235); scores f32 [T*k]; pool arrays [cap, out, in*bits/32] /
 * [cap, out, in/group]; out f32 [T, H] = sum_j scores[t*k+j] * y[t*k+j] in
 * fixed j order (reduce_pairs, fused_moe.cpp:284-298).  A slot outside
 * [0, cap) is an error. */
/* All pair outputs y[p] = expert(slots[p], x[p / k]) in parallel (double). */
static int pairs_f64(const orc_pool* pool, const int32_t* slots, int npairs, int k, const double* xd, int H, int I,
                     int group, int bits, double* y_all) {
    int err = 0;
#pragma omp parallel
    {
        double* a = (double*)malloc(sizeof(double) * I);
        if (!a) {
#pragma omp atomic write
            err = 1;
        } else {
#pragma omp for schedule(dynamic, 1)
            for (int p = 0; p < npairs; ++p)
                expert_f64(pool, slots[p], xd + (size_t)(p / k) * H, H, I, group, bits, a, y_all + (size_t)p * H);
            free(a);
        }
    }
    return err ? ORC_ENOMEM : ORC_OK;
}

int orc_fused_moe_slots(const float* x, const int32_t* slots, const float* scores, const uint32_t* gw,
                        const uint16_t* gs, const uint16_t* gb, const uint32_t* uw, const uint16_t* us,
                        const uint16_t* ub, const uint32_t* dw, const uint16_t* ds, const uint16_t* db, int T, int k,
                        int H, int I, int group, int bits, int cap, float* out) {
    if (T <= 0 || k <= 0 || H % group || I % group || (H * bits) % 32 || (I * bits) % 32) return ORC_EINVAL;
    for (int p = 0; p < T * k; ++p)
        if (slots[p] < 0 || slots[p] >= cap) return ORC_ESLOT;
    orc_pool pool = {gw, uw, dw, gs, gb, us, ub, ds, db};
    double* xd = (double*)malloc(sizeof(double) * (size_t)T * H);
    double* y = (double*)malloc(sizeof(double) * (size_t)T * k * H);
    if (!xd || !y) { free(xd); free(y); return ORC_ENOMEM; }
    for (size_t i = 0; i < (size_t)T * H; ++i) xd[i] = x[i];
    int rc = pairs_f64(&pool, slots, T * k, k, xd, H, I, group, bits, y);
    if (rc == ORC_OK) {
        for (int t = 0; t < T; ++t)
            for (int h = 0; h < H; ++h) {
                double acc = 0.0;
                for (int j = 0; j < k; ++j) acc += y[((size_t)t * k + j) * H + h] * (double)scores[t * k + j];
                out[(size_t)t * H + h] = (float)acc;
            }
    }
    free(xd); free(y);
    return rc;
}

/* Pre-MoE RMSNorm (the decoder layer's post_attention_layernorm ahead of its
 * MoE block; mlx rms_norm: x * rsqrt(mean(x^2) + eps) * w, output in bf16) in
 * the GPU kernel's canonical order: lane l of 64 sums x^2 over columns
 * [l*cpl, (l+1)*cpl) with fmaf in column order, then canon_sum64; the
 * inverse rms is 1/sqrt(ss/H + eps) with correctly rounded sqrt and division;
 * xn = bf16((x * inv) * w). */
int orc_rmsnorm_bf16(const uint16_t* x_bf16, const uint16_t* w_bf16, float eps, int T, int H, uint16_t* out,
                     float* inv_out) {
    if (T <= 0 || H % 64 || (H / 64) % 8) return ORC_EINVAL;
    int cpl = H / 64;
    for (int t = 0; t < T; ++t) {
        const uint16_t* xr = x_bf16 + (size_t)t * H;
        float a[64];
        for (int l = 0; l < 64; ++l) {
            float ss = 0.0f;
            for (int j = 0; j < cpl; ++j) {
                float v = bf16_to_f32(xr[l * cpl + j]);
                ss = fmaf(v, v, ss);
            }
            a[l] = ss;
        }
        float inv = 1.0f / sqrtf(canon_sum64(a) * (1.0f / (float)H) + eps);
        if (inv_out) inv_out[t] = inv;
        for (int c = 0; c < H; ++c)
            out[(size_t)t * H + c] = orc_f32_to_bf16((bf16_to_f32(xr[c]) * inv) * bf16_to_f32(w_bf16[c]));
    }
    return ORC_OK;
}

/* Full MoE layer (FileStreamingMoeBlock.__call__, block.py:245-1013, production
 * branch; shared expert block.py:102-109, :1009-1012):
 *   xn = rmsnorm(x) when norm_w, else x       -> bf16, GPU order (bit-exact)
 *   raw = router(xn) (+ logit_bias)           -> fp32, GPU order (bit-exact)
 *   ids, scores = topk_softmax(raw)           -> block.py:321-329
 *   local = slot_table[ids]                   -> resident_pool.py:549-580
 *   y = sum_j scores_j * expert(local_j, xn)  -> block.py:1008
 *   y += sigmoid(shared_gate(xn)) * shared(xn) -> block.py:102-109
 *   out = bf16(y (+ x if residual))
 * x is bf16 [T, H].  Outputs: out_f32 (pre-rounding), out_bf16, ids, scores,
 * slots.  Returns ORC_ESLOT when the table maps a routed expert outside
 * [0, cap). */
static int moe_layer_impl(const uint16_t* x_bf16, int T, int H, int I, int E, int k, int group, int norm_topk,
                  const uint32_t* rw, const uint16_t* rs, const uint16_t* rb, int router_bits, const float* logit_bias,
                  const int32_t* slot_table, int cap, const uint32_t* gw, const uint16_t* gs, const uint16_t* gb,
                  const uint32_t* uw, const uint16_t* us, const uint16_t* ub, const uint32_t* dw, const uint16_t* ds,
                  const uint16_t* db, int bits, const uint32_t* sh_gw, const uint16_t* sh_gs, const uint16_t* sh_gb,
                  const uint32_t* sh_uw, const uint16_t* sh_us, const uint16_t* sh_ub, const uint32_t* sh_dw,
                  const uint16_t* sh_ds, const uint16_t* sh_db, const uint32_t* sg_w, const uint16_t* sg_s,
                  const uint16_t* sg_b, int sg_bits, const uint16_t* norm_w, float norm_eps, int residual,
                  float* out_f32, uint16_t* out_bf16, int32_t* ids, float* scores, int32_t* slots,
                  const int32_t* ids_in, const float* scores_in) {
    if (T <= 0 || k <= 0 || k > E || H % group || I % group) return ORC_EINVAL;
    const uint16_t* x_raw = x_bf16;
    uint16_t* xn = NULL;
    if (norm_w) {
        xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
        if (!xn) return ORC_ENOMEM;
        int nrc = orc_rmsnorm_bf16(x_raw, norm_w, norm_eps, T, H, xn, NULL);
        if (nrc) { free(xn); return nrc; }
        x_bf16 = xn;
    }
    int rc = ORC_OK;
    if (ids_in) {
        memcpy(ids, ids_in, sizeof(int32_t) * (size_t)T * k);
        memcpy(scores, scores_in, sizeof(float) * (size_t)T * k);
    } else {
        float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
        if (!logits) { free(xn); return ORC_ENOMEM; }
        rc = orc_router_logits_f32(rw, rs, rb, logit_bias, E, H, group, router_bits, x_bf16, T, logits);
        if (rc) { free(logits); free(xn); return rc; }
        rc = orc_topk_softmax(logits, T, E, k, norm_topk, ids, scores);
        free(logits);
        if (rc) { free(xn); return rc; }
    }
    int bad = 0;
    for (int p = 0; p < T * k; ++p) {
        int e = ids[p];
        int sl = slot_table ? slot_table[e] : e;
        slots[p] = sl;
        if (sl < 0 || sl >= cap) bad = 1;
    }
    if (bad) { free(xn); return ORC_ESLOT; }
    orc_pool pool = {gw, uw, dw, gs, gb, us, ub, ds, db};
    orc_pool shp = {sh_gw, sh_uw, sh_dw, sh_gs, sh_gb, sh_us, sh_ub, sh_ds, sh_db};
    double* xd = (double*)malloc(sizeof(double) * (size_t)T * H);
    double* y = (double*)malloc(sizeof(double) * (size_t)T * k * H);
    double* ysh = (double*)malloc(sizeof(double) * (size_t)T * H);
    if (!xd || !y || !ysh) { free(xd); free(y); free(ysh); free(xn); return ORC_ENOMEM; }
    for (size_t i = 0; i < (size_t)T * H; ++i) xd[i] = bf16_to_f32(x_bf16[i]);
    rc = pairs_f64(&pool, slots, T * k, k, xd, H, I, group, bits, y);
    if (rc == ORC_OK && sh_gw) {
        int32_t* zero = (int32_t*)calloc((size_t)T, sizeof(int32_t));
        rc = zero ? pairs_f64(&shp, zero, T, 1, xd, H, I, group, bits, ysh) : ORC_ENOMEM;
        free(zero);
    }
    if (rc == ORC_OK) {
        for (int t = 0; t < T; ++t) {
            const double* xt = xd + (size_t)t * H;
            double gate = 1.0;
            if (sh_gw && sg_w) {
                double gl = 0.0;
                for (int c = 0; c < H; ++c) gl += (double)deq(sg_w, sg_s, sg_b, c, group, sg_bits) * xt[c];
                gate = 1.0 / (1.0 + exp(-gl));
            }
            for (int h = 0; h < H; ++h) {
                double acc = 0.0;
                for (int j = 0; j < k; ++j) acc += y[((size_t)t * k + j) * H + h] * (double)scores[t * k + j];
                if (sh_gw) acc += gate * ysh[(size_t)t * H + h];
                double v = acc + (residual ? (double)bf16_to_f32(x_raw[(size_t)t * H + h]) : 0.0);
                if (out_f32) out_f32[(size_t)t * H + h] = (float)v;
                if (out_bf16) out_bf16[(size_t)t * H + h] = orc_f32_to_bf16((float)v);
            }
        }
    }
    free(xd); free(y); free(ysh); free(xn);
    return rc;
}

int orc_moe_layer(const uint16_t* x_bf16, int T, int H, int I, int E, int k, int group, int norm_topk,
                  const uint32_t* rw, const uint16_t* rs, const uint16_t* rb, int router_bits, const float* logit_bias,
                  const int32_t* slot_table, int cap, const uint32_t* gw, const uint16_t* gs, const uint16_t* gb,
                  const uint32_t* uw, const uint16_t* us, const uint16_t* ub, const uint32_t* dw, const uint16_t* ds,
                  const uint16_t* db, int bits, const uint32_t* sh_gw, const uint16_t* sh_gs, const uint16_t* sh_gb,
                  const uint32_t* sh_uw, const uint16_t* sh_us, const uint16_t* sh_ub, const uint32_t* sh_dw,
                  const uint16_t* sh_ds, const uint16_t* sh_db, const uint32_t* sg_w, const uint16_t* sg_s,
                  const uint16_t* sg_b, int sg_bits, const uint16_t* norm_w, float norm_eps, int residual,
                  float* out_f32, uint16_t* out_bf16, int32_t* ids, float* scores, int32_t* slots) {
    return moe_layer_impl(x_bf16, T, H, I, E, k, group, norm_topk, rw, rs, rb, router_bits, logit_bias, slot_table,
                          cap, gw, gs, gb, uw, us, ub, dw, ds, db, bits, sh_gw, sh_gs, sh_gb, sh_uw, sh_us, sh_ub,
                          sh_dw, sh_ds, sh_db, sg_w, sg_s, sg_b, sg_bits, norm_w, norm_eps, residual, out_f32,
                          out_bf16, ids, scores, slots, NULL, NULL);
}

/* The same layer with the routing given (ids [T, k] and their combine scores):
 * checks expert math independently of near-tie routing decisions. */
int orc_moe_layer_routed(const uint16_t* x_bf16, int T, int H, int I, int E, int k, int group,
                         const int32_t* slot_table, int cap, const uint32_t* gw, const uint16_t* gs,
                         const uint16_t* gb, const uint32_t* uw, const uint16_t* us, const uint16_t* ub,
                         const uint32_t* dw, const uint16_t* ds, const uint16_t* db, int bits, const uint32_t* sh_gw,
                         const uint16_t* sh_gs, const uint16_t* sh_gb, const uint32_t* sh_uw, const uint16_t* sh_us,
                         const uint16_t* sh_ub, const uint32_t* sh_dw, const uint16_t* sh_ds, const uint16_t* sh_db,
                         const uint32_t* sg_w, const uint16_t* sg_s, const uint16_t* sg_b, int sg_bits,
                         const uint16_t* norm_w, float norm_eps, int residual, const int32_t* ids_in,
                         const float* scores_in, float* out_f32, uint16_t* out_bf16) {
    int32_t* ids = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * k);
    float* sc = (float*)malloc(sizeof(float) * (size_t)T * k);
    int32_t* sl = (int32_t*)malloc(sizeof(int32_t) * (size_t)T * k);
    int rc = (!ids || !sc || !sl) ? ORC_ENOMEM
             : moe_layer_impl(x_bf16, T, H, I, E, k, group, 1, NULL, NULL, NULL, 8, NULL, slot_table, cap, gw, gs,
                              gb, uw, us, ub, dw, ds, db, bits, sh_gw, sh_gs, sh_gb, sh_uw, sh_us, sh_ub, sh_dw,
                              sh_ds, sh_db, sg_w, sg_s, sg_b, sg_bits, norm_w, norm_eps, residual, out_f32, out_bf16,
                              ids, sc, sl, ids_in, scores_in);
    free(ids);
    free(sc);
    free(sl);
    return rc;
}

/* ------------------------------------------------- expert-major prefill */
/* Group formation (block.py:141-172): per-expert counts of the flattened
 * routes; walk experts in ascending id, skip empty ones, close a group when it
 * already holds max_group_experts experts or adding the next expert would
 * exceed max_assignments.  Writes group_start[g] (index into the expert list)
 * and returns the number of groups; experts_out lists the non-empty experts in
 * ascending order. */
int orc_expert_major_groups(const int32_t* route_ids, int n_routes, int num_experts, int max_group_experts,
                            int max_assignments, int32_t* counts, int32_t* experts_out, int32_t* n_experts_out,
                            int32_t* group_start, int32_t* group_assign) {
    if (n_routes < 0 || num_experts <= 0 || max_group_experts <= 0) return ORC_EINVAL;
    for (int e = 0; e < num_experts; ++e) counts[e] = 0;
    for (int i = 0; i < n_routes; ++i) {
        if (route_ids[i] < 0 || route_ids[i] >= num_experts) return ORC_EINVAL;
        counts[route_ids[i]]++;
    }
    int ng = 0, ne = 0, in_group = 0, assign = 0;
    for (int e = 0; e < num_experts; ++e) {
        if (counts[e] == 0) continue;
        if (in_group && (in_group >= max_group_experts || assign + counts[e] > max_assignments)) {
            group_assign[ng - 1] = assign;
            in_group = 0;
            assign = 0;
        }
        if (in_group == 0) group_start[ng++] = ne;
        experts_out[ne++] = e;
        in_group++;
        assign += counts[e];
    }
    if (ng) group_assign[ng - 1] = assign;
    *n_experts_out = ne;
    return ng;
}

/* deterministic_route_reduce (custom_kernel.py:20-118): `assignment_pos` holds
 * unique positions in the flattened [tokens, k] route table; rows of
 * `weighted` belong to those positions.  Each touched token's new value is
 * previous[token] followed by the values of its routes added one at a time in
 * ascending route-rank order, rounding after every add (to bf16 when
 * `bf16_acc`); untouched tokens keep `previous`.  In place on `out` (which
 * holds previous on entry). */
int orc_route_reduce(float* out, const float* weighted, const int32_t* assignment_pos, int n, int tokens, int hidden,
                     int k, int bf16_acc) {
    if (n < 0 || tokens <= 0 || hidden <= 0 || k <= 0) return ORC_EINVAL;
    int32_t* order = (int32_t*)malloc(sizeof(int32_t) * (n > 0 ? n : 1));
    if (!order) return ORC_ENOMEM;
    for (int i = 0; i < n; ++i) order[i] = i;
    /* insertion sort by position (positions are unique) */
    for (int i = 1; i < n; ++i) {
        int v = order[i], j = i - 1;
        while (j >= 0 && assignment_pos[order[j]] > assignment_pos[v]) { order[j + 1] = order[j]; --j; }
        order[j + 1] = v;
    }
    for (int i = 0; i < n; ++i) {
        int pos = assignment_pos[order[i]];
        if (pos < 0 || pos >= tokens * k) { free(order); return ORC_EINVAL; }
    }
    for (int i = 0; i < n; ++i) {
        int row = order[i];
        int tok = assignment_pos[row] / k;
        for (int h = 0; h < hidden; ++h) {
            float v = out[(size_t)tok * hidden + h] + weighted[(size_t)row * hidden + h];
            if (bf16_acc) v = bf16_to_f32(orc_f32_to_bf16(v));
            out[(size_t)tok * hidden + h] = v;
        }
    }
    free(order);
    return ORC_OK;
}

/* ------------------------------------------------------------- attention */
/* Full-attention block of a Qwen3-Next decoder layer on T tokens at cache
 * positions pos0.. (the MTP layer, qwen3_next_mtp.py:53; the architecture of
 * mlx-lm's / transformers' Qwen3NextAttention), in double:
 *   xn = rmsnorm(x) (bf16, orc_rmsnorm_bf16); q|gate, k, v = W xn;
 *   per head q, k: q * inv_rms(q) * q_norm (eps), rotary on dims < rope_dim
 *   (pairs (i, i + rope_dim/2), angle pos * theta^(-2i/rope_dim));
 *   token t attends to positions <= pos0 + t: cache entries < pos0 come from
 *   k_cache/v_cache (bf16 [n_kv, max_len, 256]), the batch's own from the
 *   values just computed; o = softmax(q k / sqrt(256)) v * sigmoid(gate);
 *   out = x + o_proj o.
 * k_new / v_new (optional, double [T, n_kv, 256]) receive the batch's k (after
 * norm and rotary) and v.  GQA: query head h reads kv head h / (n_heads/n_kv). */
int orc_attention_layer_f64(const uint16_t* x, int T, int H, int n_heads, int n_kv, int rope_dim, float theta,
                            float eps, const uint16_t* in_norm, const uint32_t* qw, const uint16_t* qs,
                            const uint16_t* qb, const uint32_t* kw, const uint16_t* ks, const uint16_t* kb,
                            const uint32_t* vw, const uint16_t* vs, const uint16_t* vb, const uint32_t* ow,
                            const uint16_t* os, const uint16_t* ob, int bits, const uint16_t* q_norm,
                            const uint16_t* k_norm, int pos0, const uint16_t* k_cache, const uint16_t* v_cache,
                            int max_len, double* out, double* k_new, double* v_new) {
    const int D = 256, G = n_heads / n_kv, group = 64;
    if (T <= 0 || n_kv <= 0 || n_heads % n_kv || rope_dim > D || pos0 < 0 || pos0 + T > max_len) return ORC_EINVAL;
    uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
    double* xd = (double*)malloc(sizeof(double) * (size_t)T * H);
    double* qg = (double*)malloc(sizeof(double) * (size_t)T * n_heads * 2 * D);
    double* kk = (double*)malloc(sizeof(double) * (size_t)T * n_kv * D);
    double* vv = (double*)malloc(sizeof(double) * (size_t)T * n_kv * D);
    double* att = (double*)malloc(sizeof(double) * (size_t)T * n_heads * D);
    double* sc = (double*)malloc(sizeof(double) * (size_t)(pos0 + T));
    int rc = (!xn || !xd || !qg || !kk || !vv || !att || !sc) ? ORC_ENOMEM : ORC_OK;
    if (rc == ORC_OK) rc = orc_rmsnorm_bf16(x, in_norm, eps, T, H, xn, NULL);
    if (rc == ORC_OK) {
        for (size_t i = 0; i < (size_t)T * H; ++i) xd[i] = bf16_to_f32(xn[i]);
        qgemv_f64(qw, qs, qb, n_heads * 2 * D, H, group, bits, xd, T, qg);
        qgemv_f64(kw, ks, kb, n_kv * D, H, group, bits, xd, T, kk);
        qgemv_f64(vw, vs, vb, n_kv * D, H, group, bits, xd, T, vv);
        const int half = rope_dim / 2;
        for (int t = 0; t < T; ++t) {
            const int pos = pos0 + t;
            for (int h = 0; h < n_heads + n_kv; ++h) {
                double* v = h < n_heads ? qg + ((size_t)t * n_heads + h) * 2 * D : kk + ((size_t)t * n_kv + (h - n_heads)) * D;
                const uint16_t* nw = h < n_heads ? q_norm : k_norm;
                double ss = 0.0;
                for (int d = 0; d < D; ++d) ss += v[d] * v[d];
                const double inv = 1.0 / sqrt(ss / D + (double)eps);
                double tmp[256];
                for (int d = 0; d < D; ++d) tmp[d] = v[d] * inv * (double)bf16_to_f32(nw[d]);
                for (int d = 0; d < D; ++d) {
                    double r = tmp[d];
                    if (d < rope_dim) {
                        const int i = d < half ? d : d - half;
                        const double ang = (double)pos * pow((double)theta, -(double)(2 * i) / (double)rope_dim);
                        const double partner = d < half ? -tmp[d + half] : tmp[d - half];
                        r = tmp[d] * cos(ang) + partner * sin(ang);
                    }
                    v[d] = r;
                }
            }
        }
        if (k_new) memcpy(k_new, kk, sizeof(double) * (size_t)T * n_kv * D);
        if (v_new) memcpy(v_new, vv, sizeof(double) * (size_t)T * n_kv * D);
        for (int t = 0; t < T; ++t) {
            for (int h = 0; h < n_heads; ++h) {
                const int g = h / G;
                const double* q = qg + ((size_t)t * n_heads + h) * 2 * D;
                const double* gate = q + D;
                const int L = pos0 + t + 1;
                double mx = -INFINITY;
                for (int j = 0; j < L; ++j) {
                    double dot = 0.0;
                    if (j < pos0) {
                        const uint16_t* kr = k_cache + ((size_t)g * max_len + j) * D;
                        for (int d = 0; d < D; ++d) dot += q[d] * (double)bf16_to_f32(kr[d]);
                    } else {
                        const double* kr = kk + ((size_t)(j - pos0) * n_kv + g) * D;
                        for (int d = 0; d < D; ++d) dot += q[d] * kr[d];
                    }
                    sc[j] = dot / 16.0;
                    if (sc[j] > mx) mx = sc[j];
                }
                double den = 0.0;
                for (int j = 0; j < L; ++j) { sc[j] = exp(sc[j] - mx); den += sc[j]; }
                double* o = att + ((size_t)t * n_heads + h) * D;
                for (int d = 0; d < D; ++d) o[d] = 0.0;
                for (int j = 0; j < L; ++j) {
                    const double p = sc[j] / den;
                    if (j < pos0) {
                        const uint16_t* vr = v_cache + ((size_t)g * max_len + j) * D;
                        for (int d = 0; d < D; ++d) o[d] += p * (double)bf16_to_f32(vr[d]);
                    } else {
                        const double* vr = vv + ((size_t)(j - pos0) * n_kv + g) * D;
                        for (int d = 0; d < D; ++d) o[d] += p * vr[d];
                    }
                }
                for (int d = 0; d < D; ++d) o[d] *= 1.0 / (1.0 + exp(-gate[d]));
            }
        }
        qgemv_f64(ow, os, ob, H, n_heads * D, group, bits, att, T, out);
        for (size_t i = 0; i < (size_t)T * H; ++i) out[i] += bf16_to_f32(x[i]);
    }
    free(xn); free(xd); free(qg); free(kk); free(vv); free(att); free(sc);
    return rc;
}

/* ------------------------------------------------------- Gated DeltaNet */
/* The linear-attention block of a Qwen3-Next decoder layer with per-token
 * state capture, as the reference runs it at verify time
 * (mlx_streaming/mtp/kv_cache.py:34-102 over
 * core/linear_attn/gated_delta_multistate.py:27-143), in double:
 *   xn = rmsnorm_bf16(x, in_norm); P = qkvz . xn ([n_k groups][q dk | k dk |
 *   v r*dv | z r*dv], r = n_v / n_k); ba = ba_w . xn ([n_k][b r | a r]);
 *   conv input row m_t = [q all heads | k all heads | v all heads]
 *   (conv_dim = 2 n_k dk + n_v dv); c_t = silu(sum_j conv_w[c][j] m_{t-3+j}[c])
 *   with m of positions before the batch from conv_in (3 rows, oldest first);
 *   q = c_q / sqrt(mean(c_q^2) + 1e-6) / dk, k = c_k / sqrt(mean(c_k^2) + 1e-6)
 *   / sqrt(dk) (kv_cache.py:61-63), per head;
 *   v-head h reads k-head h / r; beta = sigmoid(b), g = exp(-exp(A_log)
 *   softplus(a + dt_bias)); S <- S g; kv = S k; delta = (v - kv) beta;
 *   S <- S + delta k^T; y = S q  (S [dv][dk], gated_delta_multistate.py:74-104);
 *   o = y / sqrt(mean(y^2) + eps) * norm_w * silu(z) per v-head;
 *   out = x + out_proj o.
 * conv_rows (optional, [T][conv_dim]) receives m_t; states (optional,
 * [T][n_v][dv][dk]) the state after each token; state_in NULL = zeros. */
int orc_gdn_layer_f64(const uint16_t* x, int T, int H, int n_k, int n_v, int dk, int dv, float eps,
                      const uint16_t* in_norm, const uint32_t* pw, const uint16_t* ps, const uint16_t* pb,
                      const uint32_t* bw, const uint16_t* bs, const uint16_t* bb, const uint32_t* ow,
                      const uint16_t* os, const uint16_t* ob, int bits, const uint16_t* conv_w, const float* A_log,
                      const float* dt_bias, const uint16_t* norm_w, const double* conv_in, const double* state_in,
                      double* out, double* conv_rows, double* states) {
    const int group = 64;
    if (T <= 0 || n_k <= 0 || n_v % n_k || dk <= 0 || dv <= 0) return ORC_EINVAL;
    const int r = n_v / n_k, per_g = 2 * dk + 2 * r * dv;
    const int nq = n_k * dk, cd = 2 * nq + n_v * dv;
    const size_t ss = (size_t)n_v * dv * dk;
    uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
    double* xd = (double*)malloc(sizeof(double) * (size_t)T * H);
    double* P = (double*)malloc(sizeof(double) * (size_t)T * n_k * per_g);
    double* BA = (double*)malloc(sizeof(double) * (size_t)T * 2 * n_v);
    double* M = (double*)malloc(sizeof(double) * (size_t)(T + 3) * cd);
    double* C = (double*)malloc(sizeof(double) * (size_t)cd);
    double* S = (double*)malloc(sizeof(double) * ss);
    double* o = (double*)malloc(sizeof(double) * (size_t)T * n_v * dv);
    int rc = (!xn || !xd || !P || !BA || !M || !C || !S || !o) ? ORC_ENOMEM : ORC_OK;
    if (rc == ORC_OK) rc = orc_rmsnorm_bf16(x, in_norm, eps, T, H, xn, NULL);
    if (rc == ORC_OK) {
        for (size_t i = 0; i < (size_t)T * H; ++i) xd[i] = bf16_to_f32(xn[i]);
        qgemv_f64(pw, ps, pb, n_k * per_g, H, group, bits, xd, T, P);
        qgemv_f64(bw, bs, bb, 2 * n_v, H, group, bits, xd, T, BA);
        for (int j = 0; j < 3; ++j)
            for (int c = 0; c < cd; ++c) M[(size_t)j * cd + c] = conv_in ? conv_in[(size_t)j * cd + c] : 0.0;
        for (int t = 0; t < T; ++t) {
            double* m = M + (size_t)(t + 3) * cd;
            const double* pr = P + (size_t)t * n_k * per_g;
            for (int g = 0; g < n_k; ++g)
                for (int d = 0; d < dk; ++d) {
                    m[g * dk + d] = pr[(size_t)g * per_g + d];
                    m[nq + g * dk + d] = pr[(size_t)g * per_g + dk + d];
                }
            for (int h = 0; h < n_v; ++h)
                for (int d = 0; d < dv; ++d)
                    m[2 * nq + h * dv + d] = pr[(size_t)(h / r) * per_g + 2 * dk + (h % r) * dv + d];
            if (conv_rows) memcpy(conv_rows + (size_t)t * cd, m, sizeof(double) * cd);
        }
        if (state_in) memcpy(S, state_in, sizeof(double) * ss);
        else memset(S, 0, sizeof(double) * ss);
        for (int t = 0; t < T; ++t) {
            for (int c = 0; c < cd; ++c) {
                double acc = 0.0;
                for (int j = 0; j < 4; ++j) acc += (double)bf16_to_f32(conv_w[(size_t)c * 4 + j]) * M[(size_t)(t + j) * cd + c];
                C[c] = acc / (1.0 + exp(-acc));
            }
            for (int h = 0; h < 2 * n_k; ++h) {  /* q heads then k heads */
                double* v = C + (size_t)h * dk;
                double sq = 0.0;
                for (int d = 0; d < dk; ++d) sq += v[d] * v[d];
                const double f = 1.0 / sqrt(sq / dk + 1e-6) / (h < n_k ? (double)dk : sqrt((double)dk));
                for (int d = 0; d < dk; ++d) v[d] *= f;
            }
            const double* pr = P + (size_t)t * n_k * per_g;
            for (int h = 0; h < n_v; ++h) {
                const int gk = h / r, j = h % r;
                const double b = BA[(size_t)t * 2 * n_v + gk * 2 * r + j];
                const double a = BA[(size_t)t * 2 * n_v + gk * 2 * r + r + j];
                const double beta = 1.0 / (1.0 + exp(-b));
                const double sp = a + dt_bias[h] > 30.0 ? a + dt_bias[h] : log1p(exp(a + dt_bias[h]));
                const double gd = exp(-exp((double)A_log[h]) * sp);
                const double* q = C + (size_t)gk * dk;
                const double* k = C + nq + (size_t)gk * dk;
                const double* vv = C + 2 * nq + (size_t)h * dv;
                double* Sh = S + (size_t)h * dv * dk;
                double* y = o + ((size_t)t * n_v + h) * dv;
                for (int e = 0; e < dv; ++e) {
                    double* row = Sh + (size_t)e * dk;
                    double kv = 0.0;
                    for (int d = 0; d < dk; ++d) { row[d] *= gd; kv += row[d] * k[d]; }
                    const double delta = (vv[e] - kv) * beta;
                    double yo = 0.0;
                    for (int d = 0; d < dk; ++d) { row[d] += k[d] * delta; yo += row[d] * q[d]; }
                    y[e] = yo;
                }
                /* gated RMSNorm */
                const double* z = pr + (size_t)gk * per_g + 2 * dk + r * dv + j * dv;
                double sq = 0.0;
                for (int e = 0; e < dv; ++e) sq += y[e] * y[e];
                const double inv = 1.0 / sqrt(sq / dv + (double)eps);
                for (int e = 0; e < dv; ++e)
                    y[e] = y[e] * inv * (double)bf16_to_f32(norm_w[e]) * (z[e] / (1.0 + exp(-z[e])));
            }
            if (states) memcpy(states + (size_t)t * ss, S, sizeof(double) * ss);
        }
        qgemv_f64(ow, os, ob, H, n_v * dv, group, bits, o, T, out);
        for (size_t i = 0; i < (size_t)T * H; ++i) out[i] += bf16_to_f32(x[i]);
    }
    free(xn); free(xd); free(P); free(BA); free(M); free(C); free(S); free(o);
    return rc;
}

/* ---------------------------------------------------------------- lm_head */
/* logits = W . rmsnorm(x) (generate.py:208-217; drafter.py:20-40): xn is the
 * bf16 RMSNorm output (orc_rmsnorm_bf16, the GPU's exact operand) or x itself
 * when norm_w is NULL; W bf16 [V, H]; logits[t][v] = sum_h xn[t][h] W[v][h] in
 * double.  absdot (optional) receives sum_h |xn W|, the scale of the fp32
 * rounding error of any accumulation order. */
int orc_lm_head_f64(const uint16_t* x, int T, int H, const uint16_t* norm_w, float eps, const uint16_t* W, int V,
                    double* logits, double* absdot) {
    if (T <= 0 || H <= 0 || V <= 0) return ORC_EINVAL;
    uint16_t* xn = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)T * H);
    double* xd = (double*)malloc(sizeof(double) * (size_t)T * H);
    if (!xn || !xd) { free(xn); free(xd); return ORC_ENOMEM; }
    if (norm_w) {
        int rc = orc_rmsnorm_bf16(x, norm_w, eps, T, H, xn, NULL);
        if (rc) { free(xn); free(xd); return rc; }
    } else {
        memcpy(xn, x, sizeof(uint16_t) * (size_t)T * H);
    }
    for (size_t i = 0; i < (size_t)T * H; ++i) xd[i] = (double)bf16_to_f32(xn[i]);
#pragma omp parallel for schedule(static)
    for (int v = 0; v < V; ++v) {
        const uint16_t* wr = W + (size_t)v * H;
        for (int t = 0; t < T; ++t) {
            const double* xr = xd + (size_t)t * H;
            double acc = 0.0, aa = 0.0;
            for (int h = 0; h < H; ++h) {
                const double p = xr[h] * (double)bf16_to_f32(wr[h]);
                acc += p;
                aa += fabs(p);
            }
            logits[(size_t)t * V + v] = acc;
            if (absdot) absdot[(size_t)t * V + v] = aa;
        }
    }
    free(xn);
    free(xd);
    return ORC_OK;
}

/* ----------------------------------------------------------- acceptance */
/* accept_prefix (generate.py:338-351): longest prefix with preds[j]==drafts[j].
 * Emission (generate.py:819, :850-856):
 *   mode 0 (verify T=K: [x, d1..d_{K-1}]):  m<K -> drafts[:m]+[preds[m]];
 *          m==K -> drafts[:K]; accepted_len = min(m+1, K)
 *   mode 1 (verify T=K+1: [x, d1..dK]): drafts[:m]+[preds[m]] for m<=K;
 *          accepted_len = m+1
 * preds must hold K (mode 0) or K+1 (mode 1) entries. */
int orc_accept_greedy(const int32_t* drafts, const int32_t* preds, int K, int mode, int32_t* emitted,
                      int32_t* n_emitted, int32_t* matched, int32_t* accepted_len) {
    if (K <= 0 || (mode != 0 && mode != 1)) return ORC_EINVAL;
    int m = 0;
    while (m < K && preds[m] == drafts[m]) ++m;
    int n = 0;
    for (int j = 0; j < m; ++j) emitted[n++] = drafts[j];
    if (mode == 0) {
        if (m < K) emitted[n++] = preds[m];
        *accepted_len = (m + 1 < K) ? m + 1 : K;
    } else {
        emitted[n++] = preds[m];
        *accepted_len = m + 1;
    }
    *n_emitted = n;
    *matched = m;
    return ORC_OK;
}

/* Greedy argmax over a row (ties -> lowest index; NaN ranks lowest). */
int orc_argmax_rows(const float* logits, int rows, int V, int32_t* out) {
    if (rows <= 0 || V <= 0) return ORC_EINVAL;
    for (int r = 0; r < rows; ++r) {
        const float* l = logits + (size_t)r * V;
        int best = 0;
        for (int v = 1; v < V; ++v)
            if (better(l[v], v, l[best], best)) best = v;
        out[r] = best;
    }
    return ORC_OK;
}

/* Tree verify selection (generate.py:355-420): P paths each of K drafts;
 * preds [P, K]; winner = max matched, ties -> lowest path index
 * (generate.py:383); emission as mode 0 on the winner. */
int orc_accept_tree(const int32_t* paths, const int32_t* preds, int P, int K, int32_t* best_path, int32_t* emitted,
                    int32_t* n_emitted, int32_t* matched, int32_t* accepted_len) {
    if (P <= 0 || K <= 0) return ORC_EINVAL;
    int best = 0, bm = -1;
    for (int p = 0; p < P; ++p) {
        int m = 0;
        while (m < K && preds[p * K + m] == paths[p * K + m]) ++m;
        if (m > bm) { bm = m; best = p; }
    }
    *best_path = best;
    return orc_accept_greedy(paths + best * K, preds + best * K, K, 0, emitted, n_emitted, matched, accepted_len);
}

/* ----------------------------------------------- stochastic acceptance
 * Speculative sampling (Leviathan et al. 2023, Algorithm 1; Chen et al. 2023):
 * draft d_i is kept when u_i * q(d_i) <= p(d_i); at the first rejection the
 * token is drawn from norm(max(0, p - q)); when all K drafts are kept a bonus
 * token is drawn from p_K.  The reference has no stochastic path (its drafts
 * and acceptance are greedy, generate.py:338-351); this is the published
 * method on the reference's verify layout (K drafts, K+1 target rows).
 *
 * p and q are temperature / top-p (nucleus, Holtzman et al. 2020) transforms
 * of logits, defined on integer masses so that every order of summation gives
 * the same bits:
 *   s = (float)((1/temperature) * log2(e))          (double, then rounded)
 *   W_j = floor(2^31 * 2^z), z = (l_j - max_l) * s    (fp32 ops; 2^z below)
 *   Z = sum W_j (uint64); C = ceil(top_p * Z) (double)
 *   theta = the largest value with sum_{W_j >= theta} W_j >= C
 *   nucleus S = {j : W_j >= theta, W_j > 0}, Z_S = sum_S W_j
 *   p(j) = W_j / Z_S on S, 0 elsewhere (double division)
 * 2^z: n = rint(z), f = z - n in [-1/2, 1/2], degree-6 Taylor polynomial of
 * 2^f (coefficients (ln 2)^k / k! rounded to fp32, Horner with fmaf), scaled
 * by 2^(n + 31) exactly; W = 0 for z < -32 or NaN.  Relative error of the
 * polynomial against 2^f: < 2.5e-7.
 * Uniforms: Philox4x32-10, key (seed lo, seed hi), counter (offset lo,
 * offset hi, position i, 0x5A3D1E57): word 0 = U_i (acceptance, u = U_i 2^-32),
 * word 1 = V_i (resampling).
 * Sampling from integer masses R_j with total R: t = floor(V_i * R / 2^32)
 * (128-bit product), token = smallest j with R_0 + .. + R_j > t.
 * Residual masses: R_j = floor(2^31 * max(0, p(j) - q(j))) (double); when they
 * sum to 0 the token is drawn from p.  Without draft logits q is one-hot at
 * the draft (greedy drafting). */
static const float kExp2C[7] = {0x1p+0f, 0x1.62e43p-1f, 0x1.ebfbep-3f, 0x1.c6b08ep-5f,
                                0x1.3b2ab6p-7f, 0x1.5d87fep-10f, 0x1.430912p-13f};

static inline uint32_t sd_weight(float l, float M, float s2) {
    const float z = (l - M) * s2;
    if (!(z >= -32.0f)) return 0u;
    const float n = rintf(z);
    const float f = z - n;
    float p = kExp2C[6];
    for (int k = 5; k >= 0; --k) p = fmaf(p, f, kExp2C[k]);
    return (uint32_t)ldexpf(p, (int)n + 31);
}

float orc_sd_scale(float temperature) { return (float)((1.0 / (double)temperature) * 1.4426950408889634); }

static int cmp_u32_desc(const void* a, const void* b) {
    const uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
    return (x < y) - (x > y);
}

/* Integer masses and nucleus of one logit row (definitions above).  Returns
 * 0, or ORC_EINVAL when no logit is finite (Z = 0). */
int orc_sd_masses(const float* l, int V, float temperature, float top_p, uint32_t* W, uint32_t* theta,
                  uint64_t* zs, uint64_t* z_all) {
    if (V <= 0 || !(temperature > 0.0f)) return ORC_EINVAL;
    const float s2 = orc_sd_scale(temperature);
    float M = -INFINITY;
    for (int j = 0; j < V; ++j) M = fmaxf(M, l[j]);
    uint64_t Z = 0;
    for (int j = 0; j < V; ++j) {
        W[j] = sd_weight(l[j], M, s2);
        Z += W[j];
    }
    *z_all = Z;
    if (Z == 0) return ORC_EINVAL;
    uint64_t C = (top_p >= 1.0f) ? Z : (uint64_t)ceil((double)top_p * (double)Z);
    if (C == 0) C = 1;
    uint32_t* srt = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
    if (!srt) return ORC_ENOMEM;
    memcpy(srt, W, sizeof(uint32_t) * (size_t)V);
    qsort(srt, (size_t)V, sizeof(uint32_t), cmp_u32_desc);
    uint64_t acc = 0;
    uint32_t th = 1;
    for (int i = 0; i < V && srt[i] > 0;) {
        const uint32_t v = srt[i];
        while (i < V && srt[i] == v) acc += srt[i++];  /* every tie of v joins at once */
        if (acc >= C) { th = v; break; }
    }
    free(srt);
    uint64_t Zs = 0;
    for (int j = 0; j < V; ++j)
        if (W[j] >= th && W[j] > 0) Zs += W[j];
    *theta = th;
    *zs = Zs;
    return ORC_OK;
}

static void sd_uniforms(uint64_t seed, uint64_t offset, int i, uint32_t* U, uint32_t* Vr) {
    const uint32_t ctr[4] = {(uint32_t)offset, (uint32_t)(offset >> 32), (uint32_t)i, 0x5A3D1E57u};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    orc_philox4x32_10(ctr, key, o);
    *U = o[0];
    *Vr = o[1];
}

static int sd_pick(const uint32_t* R, int V, uint64_t total, uint32_t vr) {
    const uint64_t t = (uint64_t)(((unsigned __int128)total * ((uint64_t)vr << 32)) >> 64);
    uint64_t acc = 0;
    for (int j = 0; j < V; ++j) {
        acc += R[j];
        if (acc > t) return j;
    }
    return V - 1; /* unreachable when total = sum R */
}

/* Samples one token per row of logits [rows, V] from the temperature / top-p
 * distribution with uniform V_r of position r (the drafter's sampler). */
int orc_sample_top_p(const float* logits, int rows, int V, float temperature, float top_p, uint64_t seed,
                     uint64_t offset, int32_t* out) {
    uint32_t* W = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
    if (!W) return ORC_ENOMEM;
    for (int r = 0; r < rows; ++r) {
        uint32_t th;
        uint64_t zs, z;
        int rc = orc_sd_masses(logits + (size_t)r * V, V, temperature, top_p, W, &th, &zs, &z);
        if (rc) { free(W); return rc; }
        for (int j = 0; j < V; ++j)
            if (W[j] < th) W[j] = 0;
        uint32_t U, Vr;
        sd_uniforms(seed, offset, r, &U, &Vr);
        out[r] = sd_pick(W, V, zs, Vr);
    }
    free(W);
    return ORC_OK;
}

/* result int32 [4 + K + 1]: n_emitted, matched, accepted_len, best_path (0),
 * emitted tokens.  target [K+1, V]; draft [K, V] or NULL (one-hot drafts). */
int orc_accept_stochastic(const float* target, const float* draft, const int32_t* drafts, int K, int V,
                          float temperature, float top_p, uint64_t seed, uint64_t offset, int32_t* result) {
    if (K <= 0 || V <= 0) return ORC_EINVAL;
    const int nd = (K + 1) + (draft ? K : 0);
    uint32_t* W = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V * nd);
    uint32_t* R = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
    uint32_t th[64];
    uint64_t zs[64];
    if (!W || !R || nd > 64) { free(W); free(R); return ORC_ENOMEM; }
    for (int d = 0; d < nd; ++d) {
        const float* row = d <= K ? target + (size_t)d * V : draft + (size_t)(d - K - 1) * V;
        uint64_t z;
        int rc = orc_sd_masses(row, V, temperature, top_p, W + (size_t)d * V, &th[d], &zs[d], &z);
        if (rc) { free(W); free(R); return rc; }
    }
#define PMASS(d, j) (W[(size_t)(d) * V + (j)] >= th[d] ? W[(size_t)(d) * V + (j)] : 0u)
    int m = 0;
    for (; m < K; ++m) {
        const int dj = drafts[m];
        uint32_t U, Vr;
        sd_uniforms(seed, offset, m, &U, &Vr);
        double pp = 0.0, qq = 1.0;
        if (dj >= 0 && dj < V) {
            pp = (double)PMASS(m, dj) / (double)zs[m];
            if (draft) qq = (double)PMASS(K + 1 + m, dj) / (double)zs[K + 1 + m];
        }
        const double u = (double)U * 0x1p-32;
        if (!(pp > 0.0 && u * qq <= pp)) break;
    }
    uint32_t U, Vr;
    sd_uniforms(seed, offset, m, &U, &Vr);
    int tok;
    if (m < K) {
        uint64_t tot = 0;
        for (int j = 0; j < V; ++j) {
            const double pj = (double)PMASS(m, j) / (double)zs[m];
            double qj;
            if (draft) qj = (double)PMASS(K + 1 + m, j) / (double)zs[K + 1 + m];
            else qj = (j == drafts[m]) ? 1.0 : 0.0;
            const double r = pj - qj;
            R[j] = r > 0.0 ? (uint32_t)(r * 0x1p31) : 0u;
            tot += R[j];
        }
        if (tot == 0) {
            for (int j = 0; j < V; ++j) R[j] = PMASS(m, j);
            tot = zs[m];
        }
        tok = sd_pick(R, V, tot, Vr);
    } else {
        for (int j = 0; j < V; ++j) R[j] = PMASS(K, j);
        tok = sd_pick(R, V, zs[K], Vr);
    }
#undef PMASS
    result[0] = m + 1;
    result[1] = m;
    result[2] = m + 1;
    result[3] = 0;
    for (int j = 0; j < m; ++j) result[4 + j] = drafts[j];
    result[4 + m] = tok;
    free(W);
    free(R);
    return ORC_OK;
}

int orc_version(void) { return 1; }

/* Threads of the oracle's parallel loops (the CPU baseline is timed on all
 * cores and on one); returns the previous setting. */
int orc_set_threads(int n) {
    const int prev = omp_get_max_threads();
    if (n > 0) omp_set_num_threads(n);
    return prev;
}

