// Device-side helpers shared by the libvmi kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 vmi_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 vmi_bf8 __attribute__((ext_vector_type(8)));
typedef float vmi_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t vmi_u4 __attribute__((ext_vector_type(4)));

#define VMI_WAVE 64

// Timeline stamps for tuning builds only (compiled with -DVMI_TIMELINE): the
// first thread of a workgroup records the 100 MHz real-time counter at point
// `slot` of kernel `kid` into the buffer set by vmi_timeline_set() (one per
// translation unit), laid out [kid][workgroup < 4096][slot < 16].  The product
// build compiles these to nothing.
#ifdef VMI_TIMELINE
// The pointer sits in constant memory (a scalar load) and the stamp is a
// global store: neither makes the wave wait for its outstanding vector loads.
#define VMI_TL_DECL static __constant__ unsigned long long* vmi_tl_buf = nullptr;
#define VMI_STAMP(kid, slot)                                                                       \
    do {                                                                                           \
        if (threadIdx.x == 0 && vmi_tl_buf && blockIdx.x < 4096) {                                 \
            __attribute__((address_space(1))) unsigned long long* tl_p_ =                         \
                (__attribute__((address_space(1))) unsigned long long*)vmi_tl_buf;                \
            tl_p_[((size_t)(kid) * 4096 + blockIdx.x) * 16 + (slot)] = __builtin_amdgcn_s_memrealtime(); \
        }                                                                                          \
    } while (0)
// The same by the first lane of every wave (slot + wave index).
#define VMI_STAMP_WAVE(kid, slot)                                                                  \
    do {                                                                                           \
        if ((threadIdx.x & 63) == 0 && vmi_tl_buf && blockIdx.x < 4096) {                          \
            __attribute__((address_space(1))) unsigned long long* tl_p_ =                         \
                (__attribute__((address_space(1))) unsigned long long*)vmi_tl_buf;                \
            tl_p_[((size_t)(kid) * 4096 + blockIdx.x) * 16 + (slot) + (threadIdx.x >> 6)] =       \
                __builtin_amdgcn_s_memrealtime();                                                  \
        }                                                                                          \
    } while (0)
// The wave's hardware placement (HW_ID: CU, shader array and engine in bits
// 8..14; XCC_ID in the upper word) at point `slot`.
#define VMI_STAMP_HWID(kid, slot)                                                                  \
    do {                                                                                           \
        if (threadIdx.x == 0 && vmi_tl_buf && blockIdx.x < 4096) {                                 \
            __attribute__((address_space(1))) unsigned long long* tl_p_ =                         \
                (__attribute__((address_space(1))) unsigned long long*)vmi_tl_buf;                \
            const unsigned long long hw_ = (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 4);    \
            const unsigned long long xcc_ = (unsigned)__builtin_amdgcn_s_getreg((31 << 11) | 20);  \
            tl_p_[((size_t)(kid) * 4096 + blockIdx.x) * 16 + (slot)] = hw_ | (xcc_ << 32);         \
        }                                                                                          \
    } while (0)
#else
#define VMI_TL_DECL
#define VMI_STAMP(kid, slot) \
    do {                     \
    } while (0)
#define VMI_STAMP_HWID(kid, slot) \
    do {                          \
    } while (0)
#define VMI_STAMP_WAVE(kid, slot) \
    do {                          \
    } while (0)
#endif

__device__ __forceinline__ float vmi_bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// bf16(a) | bf16(b) << 16, both rounded to nearest even by one
// v_cvt_pk_bf16_f32 (the bits vmi_f32_to_bf16 gives for every non-NaN input).
__device__ __forceinline__ uint32_t vmi_pack_bf16x2(float a, float b) {
    typedef __bf16 vmi_bf2 __attribute__((ext_vector_type(2)));
    typedef float vmi_f2 __attribute__((ext_vector_type(2)));
    const vmi_f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, vmi_bf2));
}

// Round-to-nearest-even fp32 -> bf16 bit pattern (quiet NaN kept), branch
// free: the NaN case is a select, so a wave never splits on it.
__device__ __forceinline__ uint16_t vmi_f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    const uint32_t qnan = (u >> 16) | 0x40u;
    return (uint16_t)(((u & 0x7fffffffu) > 0x7f800000u) ? qnan : rne);
}

__device__ __forceinline__ uint32_t vmi_h2_bits(_Float16 lo, _Float16 hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// 16x16x32 f16 MFMA: D[i][j] += sum_k A[i][k] B[k][j].  Lane l supplies
// A[l%16][8*(l/16)+s] and B[8*(l/16)+s][l%16] (s = 0..7) and holds
// D[4*(l/16)+r][l%16] (r = 0..3).
__device__ __forceinline__ vmi_f4 vmi_mfma_f16(const vmi_u4& a, const vmi_u4& b, const vmi_f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(vmi_half8, a), __builtin_bit_cast(vmi_half8, b),
                                                   c, 0, 0, 0);
}
__device__ __forceinline__ vmi_f4 vmi_mfma_bf16(const vmi_u4& a, const vmi_u4& b, const vmi_f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(vmi_bf8, a), __builtin_bit_cast(vmi_bf8, b), c,
                                                    0, 0, 0);
}

// Eight 4-bit values of one packed word as MFMA f16 operands, exactly:
// halves are fp16 subnormals n * 2^-24 (n in bits 0-3) or n * 2^-20 (bits 4-7).
//   r0 = (n0, n4) * 2^-24      r1 = (n1, n5) * 2^-20
//   r2 = (n2, n6) * 2^-24      r3 = (n3, n7) * 2^-20
// so operand slot s holds column perm[s] = {0,4,1,5,2,6,3,7}[s], scaled by 16
// for s in {2,3,6,7}; the matching activation operand divides those slots by 16.
__device__ __forceinline__ vmi_u4 vmi_unpack_u4_f16(uint32_t w) {
    vmi_u4 r;
    r[0] = w & 0x000F000Fu;
    r[1] = w & 0x00F000F0u;
    uint32_t t = w >> 8;
    r[2] = t & 0x000F000Fu;
    r[3] = t & 0x00F000F0u;
    return r;
}

// Eight 4-bit values of one packed word as bf16 MFMA operands (128 + n),
// exact, in the same slot order as vmi_unpack_u4_f16 (columns
// {0,4,1,5,2,6,3,7}); the 128 * sum(activation) excess is removed by the
// caller.  bf16 0x4300 is 128.0 with a mantissa step of 1.
// The constant sits in a VGPR (materialised once: the asm has no side
// effects, so repeated copies fold), which lets each word become one
// v_and_or_b32 (a VOP3 form takes no second literal or SGPR).
__device__ __forceinline__ vmi_u4 vmi_unpack_u4_bf16_128(uint32_t w) {
    uint32_t kc;
    asm("v_mov_b32 %0, 0x43004300" : "=v"(kc));
    vmi_u4 r;
    r[0] = (w & 0x000F000Fu) | kc;
    r[1] = ((w >> 4) & 0x000F000Fu) | kc;
    r[2] = ((w >> 8) & 0x000F000Fu) | kc;
    r[3] = ((w >> 12) & 0x000F000Fu) | kc;
    return r;
}

// ---------------------------------------------------------------- DPP
// Row permutes of gfx9 DPP: xor 1 and xor 2 inside quads, mirror inside
// 8-lane half rows and 16-lane rows.  A reduction through the four leaves
// every lane of a 16-lane row holding the row result; the four rows then
// meet through readlane (uniform, no LDS traffic).
#define VMI_DPP_XOR1 0xB1
#define VMI_DPP_XOR2 0x4E
#define VMI_DPP_HALF_MIRROR 0x141
#define VMI_DPP_MIRROR 0x140

template <int CTRL>
__device__ __forceinline__ uint32_t vmi_dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float vmi_dpp_f32(float v) {
    return __uint_as_float(vmi_dpp_u32<CTRL>(__float_as_uint(v)));
}
__device__ __forceinline__ float vmi_readlane_f32(float v, int lane) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), lane));
}

// `from` shifted by a DPP row control into the lane banks (4-lane groups of
// each 16-lane row) selected by BANKS; the other lanes keep `keep`.
template <int CTRL, int BANKS>
__device__ __forceinline__ float vmi_dpp_into(float keep, float from) {
    return __uint_as_float(
        (uint32_t)__builtin_amdgcn_update_dpp((int)__float_as_uint(keep), (int)__float_as_uint(from), CTRL, 0xF, BANKS, false));
}

// Row rotate by 8 inside each 16-lane row (lane r reads lane r ^ 8), written
// only to lanes 8..15 (banks 2, 3) or 0..7 (banks 0, 1) of each row; the other
// lanes keep `keep`.
#define VMI_DPP_ROW_ROR8 0x128
__device__ __forceinline__ vmi_u4 vmi_row_swap8_hi(const vmi_u4& keep, const vmi_u4& from) {
    vmi_u4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)keep[i], (int)from[i], VMI_DPP_ROW_ROR8, 0xF, 0xC, false);
    return o;
}
__device__ __forceinline__ vmi_u4 vmi_row_swap8_lo(const vmi_u4& keep, const vmi_u4& from) {
    vmi_u4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)keep[i], (int)from[i], VMI_DPP_ROW_ROR8, 0xF, 0x3, false);
    return o;
}

// Sum over each 16-lane row (the first four steps of the canonical tree
// below); every lane of a row ends with the same value, since each step adds
// the same two partial sums on both lanes of a pair.
__device__ __forceinline__ float vmi_row_sum16(float v) {
    v = v + vmi_dpp_f32<VMI_DPP_XOR1>(v);
    v = v + vmi_dpp_f32<VMI_DPP_XOR2>(v);
    v = v + vmi_dpp_f32<VMI_DPP_HALF_MIRROR>(v);
    v = v + vmi_dpp_f32<VMI_DPP_MIRROR>(v);
    return v;
}

// Wave sum in the canonical tree shared with the CPU oracle: per 16-lane row
// v += v[l^1]; v += v[l^2]; v += v[half-mirror]; v += v[mirror]; then
// (R0 + R1) + (R2 + R3) over the rows.  Uniform result.
__device__ __forceinline__ float vmi_wave_sum_canon(float v) {
    v = v + vmi_dpp_f32<VMI_DPP_XOR1>(v);
    v = v + vmi_dpp_f32<VMI_DPP_XOR2>(v);
    v = v + vmi_dpp_f32<VMI_DPP_HALF_MIRROR>(v);
    v = v + vmi_dpp_f32<VMI_DPP_MIRROR>(v);
    const float r0 = vmi_readlane_f32(v, 0), r1 = vmi_readlane_f32(v, 16);
    const float r2 = vmi_readlane_f32(v, 32), r3 = vmi_readlane_f32(v, 48);
    return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float vmi_wave_max(float v) {
    v = fmaxf(v, vmi_dpp_f32<VMI_DPP_XOR1>(v));
    v = fmaxf(v, vmi_dpp_f32<VMI_DPP_XOR2>(v));
    v = fmaxf(v, vmi_dpp_f32<VMI_DPP_HALF_MIRROR>(v));
    v = fmaxf(v, vmi_dpp_f32<VMI_DPP_MIRROR>(v));
    const float r0 = vmi_readlane_f32(v, 0), r1 = vmi_readlane_f32(v, 16);
    const float r2 = vmi_readlane_f32(v, 32), r3 = vmi_readlane_f32(v, 48);
    return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Wave-wide maximum of an unsigned 32-bit value (uniform result): the gfx9
// row-shift / row-broadcast scan, each step one v_max_u32_dpp (0 fills the
// lanes a shift leaves empty, the identity of an unsigned max), lane 63
// holding the result.
template <int CTRL, int RM, int BM>
__device__ __forceinline__ uint32_t vmi_dpp_u32_z(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, RM, BM, true);
}
__device__ __forceinline__ uint32_t vmi_wave_max_u32(uint32_t v) {
    v = max(v, vmi_dpp_u32_z<0x111, 0xF, 0xF>(v));  // row_shr:1
    v = max(v, vmi_dpp_u32_z<0x112, 0xF, 0xF>(v));  // row_shr:2
    v = max(v, vmi_dpp_u32_z<0x113, 0xF, 0xF>(v));  // row_shr:3
    v = max(v, vmi_dpp_u32_z<0x114, 0xF, 0xE>(v));  // row_shr:4, banks 1..3
    v = max(v, vmi_dpp_u32_z<0x118, 0xF, 0xC>(v));  // row_shr:8, banks 2..3
    v = max(v, vmi_dpp_u32_z<0x142, 0xA, 0xF>(v));  // row_bcast:15, rows 1 and 3
    v = max(v, vmi_dpp_u32_z<0x143, 0xC, 0xF>(v));  // row_bcast:31, rows 2 and 3
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ uint64_t vmi_u64_max(uint64_t a, uint64_t b) { return a > b ? a : b; }

// Compare-exchange of 64-bit keys: a keeps the larger when desc.
__device__ __forceinline__ void vmi_cx64(uint64_t& a, uint64_t& b, bool desc) {
    const bool sw = desc ? (a < b) : (a > b);
    const uint64_t lo = sw ? b : a, hi = sw ? a : b;
    a = lo;
    b = hi;
}

template <int CTRL>
__device__ __forceinline__ uint64_t vmi_dpp_u64(uint64_t v) {
    const uint32_t lo = vmi_dpp_u32<CTRL>((uint32_t)v), hi = vmi_dpp_u32<CTRL>((uint32_t)(v >> 32));
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t vmi_readlane_u64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

// Wave-wide maximum of a 64-bit key (uniform result).
__device__ __forceinline__ uint64_t vmi_wave_max_u64(uint64_t v) {
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_XOR1>(v));
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_XOR2>(v));
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_HALF_MIRROR>(v));
    v = vmi_u64_max(v, vmi_dpp_u64<VMI_DPP_MIRROR>(v));
    return vmi_u64_max(vmi_u64_max(vmi_readlane_u64(v, 0), vmi_readlane_u64(v, 16)),
                       vmi_u64_max(vmi_readlane_u64(v, 32), vmi_readlane_u64(v, 48)));
}

// Order key of a float for "larger value first, NaN last": -0 is folded
// into +0, NaN maps to 0 (below -inf).
__device__ __forceinline__ uint32_t vmi_order_key(float f) {
    if (f != f) return 0u;
    uint32_t u = __float_as_uint(f);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float vmi_order_key_value(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// 64-bit rank key: value order, then lower index first.
__device__ __forceinline__ uint64_t vmi_rank_key(float f, int idx) {
    return ((uint64_t)vmi_order_key(f) << 32) | (uint32_t)(0xffffffffu - (uint32_t)idx);
}

// Power-of-two factor f with max|x| * f in (2^13, 2^14]; 1 for zero / non-finite.
__device__ __forceinline__ float vmi_fp16_range_scale(float amax) {
    if (!(amax > 0.0f) || !(amax < 3.0e38f)) return 1.0f;
    int e;
    frexpf(amax, &e);  // amax = m * 2^e, m in [0.5, 1)
    return ldexpf(1.0f, 14 - e);
}

// Strict total order used for top-k and argmax: larger value first, then lower
// index; NaN ranks below every number.
__device__ __forceinline__ bool vmi_better(float a, int ia, float b, int ib) {
    bool na = a != a, nb = b != b;
    if (na != nb) return nb;
    if (!na && a != b) return a > b;
    return ia < ib;
}

// Affine-bias term sum_g b[row][g] * X[t][g] as one bf16 MFMA: X is split into
// bf16 hi + mid + lo (24 significant bits); lane block q carries two groups:
//   A = [hi(X0), mid(X0), lo(X0), 0, hi(X1), mid(X1), lo(X1), 0]
//   B = [b0, b0, b0, 0, b1, b1, b1, 0]   (b0/b1 = low/high bf16 of one word)
__device__ __forceinline__ void vmi_split3_bf16(float x, uint32_t& hi, uint32_t& mid, uint32_t& lo) {
    hi = vmi_f32_to_bf16(x);
    const float r1 = x - vmi_bf16_to_f32(hi);
    mid = vmi_f32_to_bf16(r1);
    lo = vmi_f32_to_bf16(r1 - vmi_bf16_to_f32(mid));
}
// The two values' splits are formed together, each level by one
// v_cvt_pk_bf16_f32 (the bits of vmi_split3_bf16 for every non-NaN input).
__device__ __forceinline__ vmi_u4 vmi_bias_a_operand(float x0, float x1) {
    const uint32_t hi = vmi_pack_bf16x2(x0, x1);
    const float r0 = x0 - __uint_as_float(hi << 16), r1 = x1 - __uint_as_float(hi & 0xffff0000u);
    const uint32_t mid = vmi_pack_bf16x2(r0, r1);
    const float s0 = r0 - __uint_as_float(mid << 16), s1 = r1 - __uint_as_float(mid & 0xffff0000u);
    const uint32_t lo = vmi_pack_bf16x2(s0, s1);
    vmi_u4 r;
    r[0] = (hi & 0xffffu) | (mid << 16);
    r[1] = lo & 0xffffu;
    r[2] = (hi >> 16) | (mid & 0xffff0000u);
    r[3] = lo >> 16;
    return r;
}
__device__ __forceinline__ vmi_u4 vmi_bias_b_operand(uint32_t bb) {
    const uint32_t b0 = bb & 0xffffu, b1 = bb >> 16;
    vmi_u4 r;
    r[0] = b0 | (b0 << 16);
    r[1] = b0;
    r[2] = b1 | (b1 << 16);
    r[3] = b1;
    return r;
}

// ------------------------------------------------------- direct-to-LDS loads
// global_load_lds: lane l's `size` bytes from its own global address land at
// lds + size*l (lds is wave-uniform); vmcnt counts the copy until the bytes are
// in LDS.  The 16-byte form exists on gfx950 only, so the host pass (which
// never runs kernel code) sees an empty statement.
#if defined(__HIP_DEVICE_COMPILE__)
#define VMI_LDS_DMA16(g, lds) __builtin_amdgcn_global_load_lds((const void*)(g), (lds), 16, 0, 0)
#define VMI_LDS_DMA4(g, lds) __builtin_amdgcn_global_load_lds((const void*)(g), (lds), 4, 0, 0)
#else
#define VMI_LDS_DMA16(g, lds) ((void)0)
#define VMI_LDS_DMA4(g, lds) ((void)0)
#endif

// The same 16-byte copy as opaque inline assembly, for software pipelines:
// the compiler's wait-count pass does not see it, so it never adds a
// conservative wait for it ahead of unrelated LDS reads.  The caller orders
// it with s_waitcnt vmcnt(N) before reading the bytes (vector-memory loads
// retire in issue order) and retires its own LDS reads of a buffer before
// refilling it.  lds must be wave-uniform.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"  // m0 is clobbered on purpose
__device__ __forceinline__ void vmi_lds_dma16_opaque(const void* g, const void* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(g), "s"(m0)
                 : "memory", "m0");
#else
    (void)g;
    (void)lds;
#endif
}
// Nontemporal form, same contract: for a stream read once (no reuse through L2).
__device__ __forceinline__ void vmi_lds_dma16_opaque_nt(const void* g, const void* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(g), "s"(m0)
                 : "memory", "m0");
#else
    (void)g;
    (void)lds;
#endif
}
// The 4-byte form (lane l's dword lands at lds + 4*l), same contract.
__device__ __forceinline__ void vmi_lds_dma4_opaque(const void* g, const void* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
                 :
                 : "v"(g), "s"(m0)
                 : "memory", "m0");
#else
    (void)g;
    (void)lds;
#endif
}
#pragma clang diagnostic pop

// Waits until at most N vector-memory operations of this wave are
// outstanding.  Loads complete in issue order, so everything issued more than
// N operations ago has landed.  The builtin form is seen by the compiler's
// wait-count pass, which then treats the loads it issued itself before the
// last N as complete; it does not count copies made by inline assembly, so
// that view is never ahead of the hardware.  gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 7 and lgkmcnt 15 (no wait on them).
#define VMI_VMCNT_IMM(n) ((((n) & 15) | (((n) >> 4) << 14)) | 0x0F70)
template <int N>
__device__ __forceinline__ void vmi_vm_wait_c() {
    constexpr int n = N < 0 ? 0 : (N > 63 ? 63 : N);
    __builtin_amdgcn_s_waitcnt(VMI_VMCNT_IMM(n));
}
// Run-time count (wave-uniform); counts above 15 wait for 15, which only
// waits longer.
#define VMI_VMW1(n) case n: __builtin_amdgcn_s_waitcnt(VMI_VMCNT_IMM(n)); break;
__device__ __forceinline__ void vmi_vm_wait(int n) {
    n = __builtin_amdgcn_readfirstlane(n < 0 ? 0 : (n > 15 ? 15 : n));
    switch (n) {
        VMI_VMW1(0) VMI_VMW1(1) VMI_VMW1(2) VMI_VMW1(3) VMI_VMW1(4) VMI_VMW1(5) VMI_VMW1(6) VMI_VMW1(7)
        VMI_VMW1(8) VMI_VMW1(9) VMI_VMW1(10) VMI_VMW1(11) VMI_VMW1(12) VMI_VMW1(13) VMI_VMW1(14)
        default: __builtin_amdgcn_s_waitcnt(VMI_VMCNT_IMM(15)); break;
    }
}
#undef VMI_VMW1

// A wave-uniform int through the scalar cache (s_load).  For data written by
// an earlier kernel: the scalar cache starts empty in every kernel.
__device__ __forceinline__ int32_t vmi_sload_i32(const int32_t* p) {
    return *(const __attribute__((address_space(4))) int32_t*)(uintptr_t)p;
}

// ---------------------------------------------------------- buffer loads
// Raw buffer resource over [base, base + bytes): loads past `bytes` return 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t vmi_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// Raw-buffer range checks use the per-lane offset: a lane whose offset is
// VMI_OOB reads zeros without touching memory.
#define VMI_OOB 0x80000000u
__device__ __forceinline__ vmi_u4 vmi_bload_b128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 0);
    vmi_u4 o;
    o[0] = v[0];
    o[1] = v[1];
    o[2] = v[2];
    o[3] = v[3];
    return o;
}
// Nontemporal form (streamed data that is read once).
__device__ __forceinline__ vmi_u4 vmi_bload_b128_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, 2);
    vmi_u4 o;
    o[0] = v[0];
    o[1] = v[1];
    o[2] = v[2];
    o[3] = v[3];
    return o;
}
__device__ __forceinline__ uint2 vmi_bload_b64_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 2);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t vmi_bload_b32_nt(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 2);
}
__device__ __forceinline__ uint2 vmi_bload_b64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t vmi_bload_b32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
}
// Coherent forms (cache policy sc1: device-scope coherence, the bit the
// compiler sets on agent-scope atomic loads) for data that other workgroups
// of the same kernel wrote with agent-scope stores.  Unlike atomic loads they
// are ordinary loads to the compiler, so a batch of them is issued back to
// back instead of one wait per load.
#define VMI_CP_SC1 0x10
__device__ __forceinline__ uint32_t vmi_bload_b32_coh(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, VMI_CP_SC1);
}
__device__ __forceinline__ uint2 vmi_bload_b64_coh(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, VMI_CP_SC1);
    return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ vmi_u4 vmi_bload_b128_coh(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)voff, (int)soff, VMI_CP_SC1);
    vmi_u4 o;
    o[0] = v[0];
    o[1] = v[1];
    o[2] = v[2];
    o[3] = v[3];
    return o;
}
// Buffer store of 16 bytes; a lane whose offset is VMI_OOB (past the
// resource's range) stores nothing, so a predicated store needs no branch.
__device__ __forceinline__ void vmi_bstore_b128(const vmi_u4& v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, (int)soff, 0);
}
// The same for 8 bytes.
__device__ __forceinline__ void vmi_bstore_b64(uint2 v, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b64((uint32_t __attribute__((ext_vector_type(2)))){v.x, v.y}, r, (int)voff,
                                          (int)soff, 0);
}
// Nontemporal form, for data the next kernel reads once.
__device__ __forceinline__ void vmi_bstore_b128_nt(const vmi_u4& v, __amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)voff, (int)soff, 2);
}
__device__ __forceinline__ uint32_t vmi_bload_b16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)voff, (int)soff, 0);
}

// KV cache of the attention layers: per kv head, blocks of 32 positions x 256
// dims (8192 bf16), each in the operand order of the attention kernel's MFMAs
// (vmi.h, vmi_attention_layer, states the element formulas).
constexpr int VMI_KV_BLOCK = 32;
__device__ __forceinline__ size_t vmi_kv_block(int g, int max_len, int pos) {
    return ((size_t)g * (max_len / VMI_KV_BLOCK) + pos / VMI_KV_BLOCK) * (size_t)(VMI_KV_BLOCK * 256);
}
__device__ __forceinline__ int vmi_k_elem(int kt, int d) {
    const int nl = 4 * (kt >> 3) + (kt & 3), a = (kt >> 2) & 1;
    return (((a * 8 + (d >> 5)) * 64 + ((d >> 3) & 3) * 16 + nl) << 3) + (d & 7);
}
__device__ __forceinline__ int vmi_v_elem(int kt, int d) {
    return ((((d >> 4) * 64 + (kt >> 3) * 16 + (d & 15)) << 3) + (kt & 7));
}
