/*
 * vmi.h -- C ABI of the MI355X speculative-decode MoE library (libvmi.so).
 *
 * Plain pointers, sizes and a hipStream_t passed as void*.  No exceptions cross
 * this boundary: every entry point returns VMI_OK (0) or a negative status and
 * records a message retrievable with vmi_last_error() (thread-local).
 * All device pointers must be contiguous row-major buffers on the current HIP
 * device.  Calls are stream-ordered and asynchronous: they never synchronise the
 * host.  Errors the device detects while running (a routed slot outside the
 * pool, for instance) are OR-ed into the workspace status word; read them with
 * vmi_workspace_status().
 *
 * Packed weight format (MLX affine, LSB-first): a projection stack with n
 * matrices of shape [out, in] is three arrays
 *   w  uint32 [n, out, in*bits/32]   value of column c sits at bits (c*bits)%32
 *                                    of word (c*bits)/32 of its row
 *   s  uint16 [n, out, in/group]     bf16 bit patterns of the scales
 *   b  uint16 [n, out, in/group]     bf16 bit patterns of the biases
 * and dequantises to w = q * s + b (fused_moe.cpp:131-145).
 */
#ifndef VMI_H_
#define VMI_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum vmi_status {
    VMI_OK = 0,
    VMI_ERR_INVALID = -1,     /* bad pointer, shape or argument */
    VMI_ERR_UNSUPPORTED = -2, /* valid but not built (bits, group, shape) */
    VMI_ERR_HIP = -3,         /* a HIP runtime call failed */
    VMI_ERR_WORKSPACE = -4    /* workspace missing or too small */
};

enum vmi_dtype { VMI_F32 = 0, VMI_BF16 = 1 };

/* Device-side status bits (vmi_workspace_status). */
#define VMI_STATUS_BAD_SLOT 0x1u   /* a routed slot was outside [0, cap) */
#define VMI_STATUS_BAD_ROUTE 0x2u  /* router produced a non-finite logit */
#define VMI_STATUS_BAD_POS 0x4u    /* a device-side position outside [0, max_len - T] */
#define VMI_STATUS_BAD_RECORD 0x8u /* an acceptance record outside what vmi_spec_commit allows */
#define VMI_STATUS_WAIT_GAVE_UP 0x10u /* a wait of vmi_accept_stochastic / vmi_sample_top_p outlasted its bound */
#define VMI_STATUS_BAD_LOGITS 0x20u   /* a logit row of those calls had no finite value */

/* Last error message of the calling thread ("" when none). */
const char* vmi_last_error(void);
/* ABI version; bumped on any incompatible change. */
int vmi_version(void);

/* One affine-quantised projection stack (see header comment). */
typedef struct vmi_qmat {
    const uint32_t* w;
    const uint16_t* s;
    const uint16_t* b;
} vmi_qmat;

/* ------------------------------------------------------------------------
 * vmi_fused_moe_slots -- replaces fused_moe_slots
 *   native/ext/compute/fused_moe.h:18-23 (declaration),
 *   native/ext/compute/fused_moe.cpp:514-556, 635-664 (primitive + factory),
 *   native/ext/bindings.cpp:300-320 (Python binding).
 * Same argument meaning: x [T, hidden] (x_dtype VMI_F32 as the reference's
 * caller passes, native_moe.py:481, or VMI_BF16), local_slots int32 [T*k]
 * token-major (token = pair / k, fused_moe.cpp:235), scores f32 [T*k],
 * gate/up stacks [cap, inter, hidden], down stack [cap, hidden, inter],
 * out [T, hidden] in out_dtype = sum_j scores[t*k+j] * expert_{slot}(x_t)
 * (SwiGLU expert: g*sigmoid(g)*u then down; fixed j order as reduce_pairs).
 * Arithmetic: the reference operator's fp32 throughout (x widened to fp32 -
 * exactly, for bf16 x - weights q*s + b, activations and pair outputs;
 * relative error about 1e-6 against a float64 evaluation).  The pool stacks
 * keep the reference's layout.
 * Supported: bits == 4, group == 64, T*k <= 160, T <= 16,
 * hidden in {512, 1024, 2048}, inter a multiple of 64 up to 512.
 * The reference raises on shape mismatch (fused_moe.cpp:522-524); this
 * returns VMI_ERR_INVALID.  A slot outside [0, cap) contributes zero and sets
 * VMI_STATUS_BAD_SLOT.
 * workspace: device memory of vmi_fused_moe_slots_workspace_bytes(T, k,
 * hidden, inter) bytes whose first 4 bytes (the status word) are zero before
 * its first use; it may be reused by later calls on the same stream but never
 * by two calls in flight at once.
 * ------------------------------------------------------------------------ */
size_t vmi_fused_moe_slots_workspace_bytes(int T, int k, int hidden, int inter);
int vmi_fused_moe_slots(const void* x, int x_dtype, const int32_t* local_slots, const float* scores,
                        vmi_qmat gate, vmi_qmat up, vmi_qmat down, int T, int k, int hidden, int inter, int group,
                        int bits, int cap, void* out, int out_dtype, void* workspace, size_t workspace_bytes,
                        void* stream);

/* ------------------------------------------------------------------------
 * vmi_fused_moe_staged -- replaces fused_moe_staged, the slot-less sibling
 *   native/ext/compute/fused_moe.h:11-16 (declaration),
 *   native/ext/compute/fused_moe.cpp:443-504, 605-633 (primitive + factory),
 *   native/ext/bindings.cpp:31-50 (Python binding).
 * The weight stacks hold one pre-sliced matrix per (token, rank) pair: pair
 * p = t*k + j reads matrix p (gate/up [T*k, inter, hidden], down
 * [T*k, hidden, inter]); otherwise as vmi_fused_moe_slots with
 * local_slots[p] = p, including the workspace
 * (vmi_fused_moe_slots_workspace_bytes).
 * ------------------------------------------------------------------------ */
int vmi_fused_moe_staged(const void* x, int x_dtype, const float* scores, vmi_qmat gate, vmi_qmat up,
                         vmi_qmat down, int T, int k, int hidden, int inter, int group, int bits, void* out,
                         int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * vmi_moe_layer -- one full routed-MoE layer on a verify batch; replaces the
 * production branch of FileStreamingMoeBlock.__call__
 *   mlx_streaming/core/moe/block.py:245-1013 (router :251-253, softmax/top-k/
 *   renorm :321-329, pool acquire -> local slots :680-684, SwitchGLU expert
 *   compute compute.py:145-170, combine :1008, shared expert :102-109,
 *   :1009-1012), and the MTP layer's StreamingMTPMoE.__call__
 *   mlx_streaming/mtp/qwen3_next_mtp.py:122-137.
 * Steps: xn = x, or with norm_weight the pre-MoE RMSNorm
 * xn = bf16(x * (1/sqrt(mean(x^2) + norm_eps)) * norm_weight) (the decoder
 * layer's post_attention_layernorm ahead of its MoE block); raw = router(xn)
 * (+ logit_bias); ids = top-k of raw (logit
 * descending, ties to the lower expert id); scores = softmax over the k
 * (norm_topk_prob) or over all experts; slot = slot_table[id] (identity when
 * NULL); out = sum_j scores_j * expert_slot(xn) + sigmoid(shared_gate(xn)) *
 * shared(xn) (+ residual).  x, residual and out are bf16 [T, hidden]; out must
 * not alias x.  ids_out / scores_out (may be NULL) receive [T, k].
 * Supported: expert bits 4, router/shared-gate bits 4 or 8, group 64,
 * T <= 16, num_experts <= 1024, top_k <= 16, hidden/inter as above.
 * ------------------------------------------------------------------------ */
typedef struct vmi_moe_layer_desc {
    int hidden, inter, num_experts, top_k, group, bits;
    int norm_topk_prob;
    int router_bits;              /* 4 or 8 */
    int cap;                      /* pool slots in gate/up/down */
    vmi_qmat router;              /* [1, num_experts, hidden] */
    const float* router_logit_bias; /* [num_experts] added to raw logits, or NULL */
    const int32_t* slot_table;    /* [num_experts] expert -> pool slot, or NULL */
    vmi_qmat gate, up, down;      /* pool stacks [cap, ...] in the kernels' layouts (below) */
    vmi_qmat shared_gate, shared_up, shared_down; /* [1, ...], same layouts; shared_gate.w == NULL: none */
    vmi_qmat shared_expert_gate;  /* [1, 1, hidden]; .w == NULL: gate fixed to 1 */
    int shared_expert_gate_bits;  /* 4 or 8 */
    const uint16_t* norm_weight;  /* [hidden] bf16 RMSNorm weight, or NULL: no norm */
    float norm_eps;
    const void* prefill_tables;   /* vmi_moe_prefill_tables() of these pools, or NULL (vmi_moe_prefill only) */
} vmi_moe_layer_desc;
/* Pool layouts of vmi_moe_layer / vmi_moe_prefill (the packed values, scales
 * and biases are the reference's; only their order in memory differs, and
 * vates_amd/moe.py re-lays the reference's stacks at load time):
 *   gate, up (MFMA-major): words [cap, inter/64, 4, hidden/128, 64, 4] - block
 *     (c, w, m), entry l = 16 q + r holds the 16 bytes at byte 64 m + 16 q of
 *     row 64 c + 16 w + r of the reference's [cap, inter, hidden/8] words;
 *     scales and biases [cap, inter, hidden/64] as in the reference;
 *   down (group-major): words [cap, inter/64, hidden, 8] - quantisation group
 *     g of row h; scales and biases [cap, inter/64, hidden]. */

size_t vmi_moe_layer_workspace_bytes(int T, int top_k, int hidden, int inter, int num_experts);
int vmi_moe_layer(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* residual,
                  uint16_t* out, int32_t* ids_out, float* scores_out, void* workspace, size_t workspace_bytes,
                  void* stream);

/* ------------------------------------------------------------------------
 * vmi_moe_layer_noalloc -- vmi_moe_layer without a workspace argument and
 * without any allocation: no counterpart in the reference.  It is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The same kernels run on a
 * static device array of 16 MiB per GPU (held until the process ends, looked
 * up once per device); shapes whose workspace
 * (vmi_moe_layer_workspace_bytes) exceeds it are rejected with
 * VMI_ERR_UNSUPPORTED.  Every call on one GPU shares that array and leaves
 * its contents behind: calls that overlap on one GPU (two streams, two
 * threads) race and must be serialised by the caller.  status: a device word
 * that receives the VMI_STATUS_* bits OR-ed in (the caller clears it), or
 * NULL to drop them.  Other arguments as vmi_moe_layer.
 * ------------------------------------------------------------------------ */
int vmi_moe_layer_noalloc(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* residual,
                          uint16_t* out, int32_t* ids_out, float* scores_out, uint32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * vmi_moe_prefill -- the same layer on a long prompt, expert-major; replaces
 * FileStreamingMoeBlock._expert_major_forward
 *   mlx_streaming/core/moe/block.py:111-243 (histogram + argsort of routed
 *   experts, per-expert gathers, SwitchGLU per group, weighted scatter) and
 *   its deterministic reduce core/moe/custom_kernel.py:20-118.
 * With every expert resident there is no group bound: one pass sorts the T*k
 * routes by pool slot and runs grouped MFMA GEMMs over 128-route tiles of each
 * slot (gate/up + SwiGLU, then down); the shared expert is a dense GEMM over
 * all tokens.  Every (token, rank) result has its own row and the combine adds
 * ranks 0..k-1, then the gated shared expert, in fp32 in that order: the output
 * is deterministic.  Router logits come from an MFMA GEMM (fp32 accumulation in
 * the matrix cores' order), so routed ids can differ from vmi_moe_layer's at
 * near-ties of the k-th logit.
 * desc as vmi_moe_layer (hidden 512, 1024 or 2048; inter a multiple of 64;
 * num_experts a multiple of 64 up to 1024; top_k <= 16; cap <= 1024);
 * T <= 65536; x, residual, out bf16 [T, hidden].  workspace:
 * vmi_moe_prefill_workspace_bytes(...) bytes (first 4 bytes: the status word,
 * zero before first use).
 * ------------------------------------------------------------------------ */
size_t vmi_moe_prefill_workspace_bytes(int T, int top_k, int hidden, int inter, int num_experts, int cap,
                                       int router_bits);
int vmi_moe_prefill(const vmi_moe_layer_desc* desc, const uint16_t* x, int T, const uint16_t* residual,
                    uint16_t* out, int32_t* ids_out, float* scores_out, void* workspace, size_t workspace_bytes,
                    void* stream);

/* ------------------------------------------------------------------------
 * vmi_moe_prefill_tables -- the fp16 dequantisation tables vmi_moe_prefill's
 * expert GEMMs read, for every pool slot and the shared expert, built once
 * from the pools' scales and biases.  No counterpart in the reference: a
 * derived form of the pools, as their MFMA-major order is.  With
 * desc->prefill_tables pointing at them, vmi_moe_prefill no longer builds the
 * touched experts' tables in its workspace on every call.  They follow the
 * pools' contents: a caller that rewrites pool slots builds them again.
 * Per weight row: P, the row's power of two (bounded by its largest scale and
 * bias), 2^(24-P) as f32, and per quantisation group the fp16 pair
 * (scale 2^P, bias 2^(P-24)).  tables: vmi_moe_prefill_tables_bytes(hidden,
 * inter, cap) bytes, 16-byte aligned; desc as vmi_moe_prefill.
 * ------------------------------------------------------------------------ */
size_t vmi_moe_prefill_tables_bytes(int hidden, int inter, int cap);
int vmi_moe_prefill_tables(const vmi_moe_layer_desc* desc, void* tables, size_t bytes, void* stream);

/* Reads and clears the device status word of a workspace (synchronises the
 * stream).  *flags receives VMI_STATUS_* bits. */
int vmi_workspace_status(void* workspace, void* stream, uint32_t* flags);

/* ------------------------------------------------------------------------
 * vmi_dequant_affine -- materialise w = q*s + b as f32 [rows, cols]
 * (qvalue, fused_moe.cpp:131-145).  Used to check dequantisation bit-exactly.
 * bits in {4, 8}; cols*bits % 32 == 0; cols % group == 0.
 * ------------------------------------------------------------------------ */
int vmi_dequant_affine(vmi_qmat m, int rows, int cols, int group, int bits, float* out, void* stream);

/* ------------------------------------------------------------------------
 * vmi_lm_head -- logits = weight . rmsnorm(x) over the whole vocabulary with
 * the per-token argmax fused in; replaces the verify forward's tail
 *   mlx_streaming/mtp/generate.py:208-217 (H_for_logits = inner.norm(h);
 *   logits = model.lm_head(H_for_logits)) and :756 (preds = mx.argmax of the
 *   verify logits), and the draft step's argmax
 *   mlx_streaming/mtp/drafter.py:20-40 (d = int(mx.argmax(lg))).
 * x bf16 [T, hidden]; norm_weight bf16 [hidden], or NULL for no norm (then x
 * is used as given); the norm is bf16(x * 1/sqrt(mean(x^2) + norm_eps) * w).
 * weight bf16 [vocab, hidden] (a tied embedding or the head).  Outputs, each
 * optional: logits f32 [T, vocab]; argmax int32 [T] and max_logit f32 [T],
 * the first maximum of each row (ties to the lower vocabulary row, NaN
 * never wins - mx.argmax's rule); top_prob f32 [T], the softmax probability
 * of the argmax, 1 / sum_j exp(l_j - max l) (fp32 running maxima and sums
 * merged in a fixed order), the per-draft confidence of
 * mlx_streaming/mtp/drafter.py:42-62 (conf *= softmax(lg)[d]).
 * Accumulation is fp32 (bf16 MFMA).
 * Supported: T <= 16, hidden a multiple of 512 up to 2048, pointers 16-byte
 * aligned.  workspace (required when argmax, max_logit or top_prob is requested):
 * vmi_lm_head_workspace_bytes(T, vocab) bytes, all zero before the first
 * call and left zero by every call; one call in flight per workspace.
 * ------------------------------------------------------------------------ */
size_t vmi_lm_head_workspace_bytes(int T, int vocab);
int vmi_lm_head(const uint16_t* x, int T, int hidden, const uint16_t* norm_weight, float norm_eps,
                const uint16_t* weight, int vocab, float* logits, int32_t* argmax, float* max_logit,
                float* top_prob, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * vmi_head_tiles / vmi_lm_head_tiled -- no counterpart in the reference: the
 * head re-laid once (at load) for callers that run it every decode step.
 * vmi_head_tiles copies a row-major bf16 [vocab, hidden] head into
 * vmi_head_tiles_bytes(vocab, hidden) bytes of tile-major order: element
 * (v, h) at ((v / 16) * (hidden / 128) + h / 128) * 2048 + (v % 16) * 128 +
 * h % 128, rows past vocab (up to a multiple of 16) zero; out must not alias
 * weight.  vmi_lm_head_tiled is vmi_lm_head on that copy (same arguments,
 * results bit for bit): each of its 4 KB weight chunks is contiguous, which
 * the kernel's LDS DMA streams faster than four rows' 256-byte runs.
 * ------------------------------------------------------------------------ */
size_t vmi_head_tiles_bytes(int vocab, int hidden);
int vmi_head_tiles(const uint16_t* weight, int vocab, int hidden, uint16_t* out, void* stream);
int vmi_lm_head_tiled(const uint16_t* x, int T, int hidden, const uint16_t* norm_weight, float norm_eps,
                      const uint16_t* tiles, int vocab, float* logits, int32_t* argmax, float* max_logit,
                      float* top_prob, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * vmi_qgemv -- y = W x for a small batch of tokens with an affine-quantised W
 * (the reference's quantized Linear layers: QuantizedLinear of mlx, as used
 * by the MTP fc and attention projections, qwen3_next_mtp.py:28-30, 40-53).
 * x bf16 [T, K]; W [N, K] packed (bits 4 or 8, group 64); out f32 [T, N]
 * and/or out_bf16 = bf16(y + residual) [T, N] (residual bf16 or NULL).
 * T <= 16 (launched in pieces of 8 tokens), min(T, 8)*K <= 32768, K a
 * multiple of 64.
 * ------------------------------------------------------------------------ */
int vmi_qgemv(const uint16_t* x, int T, int K, vmi_qmat w, int N, int bits, int group, float* out,
              const uint16_t* residual, uint16_t* out_bf16, void* stream);

/* ------------------------------------------------------------------------
 * vmi_attention_layer -- the full-attention block of a Qwen3-Next decoder
 * layer on a verify batch or a draft step: out = x + attn(rmsnorm(x)).
 * Replaces the attention half of mlx-lm's Qwen3NextDecoderLayer as the MTP
 * layer runs it (mlx_streaming/mtp/qwen3_next_mtp.py:53, mtp_step :60-63) and
 * the main model's full-attention layers (generate.py:101-220).
 * q_proj emits [q | gate] per head (n_heads x 2 x head_dim rows); q and k get
 * a per-head RMSNorm (q_norm, k_norm weights over head_dim), then the rotary
 * embedding on their first rope_dim dims (pairs (i, i + rope_dim/2),
 * angle pos * rope_theta^(-2i/rope_dim)); k and v are appended as bf16 to the
 * caches at positions pos0 .. pos0+T-1; token t attends to cache positions
 * <= pos0 + t with softmax(q k / sqrt(head_dim)); the result times
 * sigmoid(gate) goes through o_proj and is added to x.
 * k_cache, v_cache: bf16, per kv head max_len / 32 blocks of 32 positions x
 * head_dim (8192 elements), max_len a multiple of 32.  Inside a block,
 * position kt and dim d are stored at
 *   keys:   ((a*8 + (d>>5))*64 + ((d>>3)&3)*16 + nl)*8 + (d&7),
 *           nl = 4*(kt>>3) + (kt&3), a = (kt>>2)&1
 *   values: (((d>>4)*64 + (kt>>3)*16 + (d&15))*8 + (kt&7))
 * (the operand order of the kernel's matrix instructions: every load is a
 * contiguous 1 KB).  Positions >= pos0 + T are never used.  head_dim 256;
 * T * n_heads / n_kv_heads <= 64; norm weights are the multipliers applied
 * (a checkpoint's zero-centred weights plus one).  Keys are processed in
 * chunks of 256, 288 or 320 at fixed positions (the length set by max_len,
 * n_kv_heads and the device's CU count: the shortest that gives every chunk a
 * CU) and merged in a fixed order, so a token's result does not depend on
 * the batch it is verified in (bit for bit) for a given cache capacity.
 * pos_device (int32 on the device, or NULL): when set, the batch position is
 * read from it when the kernels run instead of pos0 (a captured graph replays
 * with positions that advance on the device); a value outside
 * [0, max_len - T] is clamped into it and sets VMI_STATUS_BAD_POS in the
 * workspace's status word (vmi_workspace_status), and the chunk grid covers
 * the whole capacity.  workspace: vmi_attention_layer_workspace_bytes(T,
 * hidden, n_heads, n_kv_heads, max_len) bytes whose first 4 bytes (the
 * status word) are zero before its first use.
 * ------------------------------------------------------------------------ */
typedef struct vmi_attn_layer_desc {
    int hidden, n_heads, n_kv_heads, head_dim, rope_dim;
    float rope_theta, norm_eps;
    int bits, group;
    const uint16_t* input_norm;   /* [hidden] */
    vmi_qmat q_proj, k_proj, v_proj, o_proj;
    const uint16_t* q_norm;       /* [head_dim] */
    const uint16_t* k_norm;       /* [head_dim] */
} vmi_attn_layer_desc;

size_t vmi_attention_layer_workspace_bytes(int T, int hidden, int n_heads, int n_kv_heads, int max_len);
int vmi_attention_layer(const vmi_attn_layer_desc* desc, const uint16_t* x, int T, int pos0,
                        const int32_t* pos_device, uint16_t* k_cache, uint16_t* v_cache, int max_len, uint16_t* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * vmi_gdn_layer -- the Gated DeltaNet (linear attention) block of a
 * Qwen3-Next decoder layer on a verify batch or decode step, capturing the
 * state after every token: out = x + gdn(rmsnorm(x)).  Replaces mlx-lm's
 * Qwen3NextGatedDeltaNet as the reference patches it for verification
 * (mlx_streaming/mtp/kv_cache.py:34-102: per-token [conv, ssm] checkpoints
 * from the multistate kernel, core/linear_attn/gated_delta_multistate.py:
 * 27-143) and its commit (commit_verified_prefix, kv_cache.py:222-251).
 * in_proj_qkvz rows per k-head group: [q dk | k dk | v r*dv | z r*dv]
 * (r = n_v / n_k); in_proj_ba per group: [b r | a r]; conv input row =
 * [q of all k-heads | k of all k-heads | v of all v-heads] (conv_dim =
 * 2 n_k dk + n_v dv), causal depthwise conv of width 4 (conv_weight bf16
 * [conv_dim][4], tap 3 = the current position) and SiLU; q and k of each
 * head are divided by sqrt(mean(.^2) + 1e-6) and scaled by 1/dk and
 * 1/sqrt(dk); beta = sigmoid(b), g = exp(-exp(A_log) softplus(a + dt_bias));
 * per v-head (reading k-head h / r) with state S [dv][dk] in fp32:
 *   S <- g S;  delta = beta (v - S k);  S <- S + delta k^T;  y = S q;
 * o = y / sqrt(mean(y^2) + norm_eps) * norm_weight * silu(z) per v-head;
 * out = x + out_proj o.
 * conv_ring: bf16 [32][conv_dim]; row p % 32 holds the conv input of
 * position p.  state_ring: f32 [n_slots][n_v][dv][dk]; slot p % n_slots holds
 * the state before position p.  A call at positions pos0..pos0+T-1 reads
 * conv rows pos0-3..pos0-1 and state slot pos0 % n_slots (zeros at pos0 = 0)
 * and writes conv rows and the state after each token (slots pos0+1 ..
 * pos0+T); n_slots >= T + 1.  Committing m accepted positions is continuing
 * at pos0 + m: nothing is copied.  head dims 128, T <= 8.  workspace:
 * vmi_gdn_layer_workspace_bytes(T, hidden, n_k_heads, n_v_heads) bytes.
 * A T-token call equals T one-token calls bit for bit.  pos_device (int32 on
 * the device, or NULL): when set, pos0 is read from it when the kernels run.
 * ------------------------------------------------------------------------ */
typedef struct vmi_gdn_layer_desc {
    int hidden, n_k_heads, n_v_heads, head_k_dim, head_v_dim;
    float norm_eps;
    int bits, group;
    const uint16_t* input_norm;   /* [hidden] */
    vmi_qmat in_proj_qkvz, in_proj_ba, out_proj;
    const uint16_t* conv_weight;  /* [conv_dim][4] bf16 */
    const float* A_log;           /* [n_v_heads] */
    const float* dt_bias;         /* [n_v_heads] */
    const uint16_t* norm_weight;  /* [head_v_dim] */
} vmi_gdn_layer_desc;

size_t vmi_gdn_layer_workspace_bytes(int T, int hidden, int n_k_heads, int n_v_heads);
int vmi_gdn_layer(const vmi_gdn_layer_desc* desc, const uint16_t* x, int T, int pos0, const int32_t* pos_device,
                  uint16_t* conv_ring, float* state_ring, int n_slots, uint16_t* out, void* workspace,
                  size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Tree verification: the P paths of a draft tree, each [x, d1 .. d_{span-1}]
 * at positions pos0 .. pos0 + span - 1 over the shared caches, verified in one
 * forward and the winning path committed afterwards.  Replaces
 * tree_verify_step's batched forward over tiled caches and commit_tree_row
 * (mlx_streaming/mtp/generate.py:355-420, kv_cache.py:283-316).
 *
 * vmi_attention_tree -- vmi_attention_layer over x bf16 [paths * span,
 * hidden] (path p's rows p*span ..): every path's token j attends to the cache
 * below pos0 and to its own path's tokens 0..j; the caches are only read, and
 * each path's new keys and values go to tree_kv bf16
 * [paths][n_kv_heads][2][span][256] (keys, then values; plain dims).  A
 * path's rows equal what vmi_attention_layer gives its tokens as a chain, bit
 * for bit.  paths * span <= 16, span <= 8.  workspace:
 * vmi_attention_tree_workspace_bytes(paths, span, ...) bytes.
 *
 * vmi_gdn_tree -- vmi_gdn_layer over the same layout: each path starts from
 * the state before pos0 and the conv rows below pos0; the rings are only
 * read; the conv inputs go to tree_conv bf16 [paths * span][conv_dim] and
 * each token's recurrence inputs to tree_side f32 [paths * span][n_k * 128 +
 * n_v * 128 + 2 n_v] (normalised k of every key head, v of every value head,
 * (g, beta) of every value head).  Rows equal vmi_gdn_layer's per path, bit
 * for bit.  workspace: vmi_gdn_layer_workspace_bytes(paths * span, ...).
 *
 * vmi_tree_commit -- after vmi_accept_greedy (mode 0, P paths): for the
 * record's winning path w and accepted length acc, writes into every layer of
 * the table (device memory, n_layers entries) the entries of positions pos0
 * .. pos0 + acc - 1: attention keys/values from tree_kv into the caches;
 * Gated DeltaNet conv inputs into the conv ring and the state before
 * pos0 + acc (the state before pos0 with path w's first acc tokens applied,
 * the same arithmetic as vmi_gdn_layer) into ring slot (pos0 + acc) %
 * n_slots.  pos0 from pos_device when set (read before vmi_spec_commit moves
 * it).  max_heads: the largest n_kv_heads / n_v_heads of the table (<= 64);
 * paths, span: the tree's shape (the table's buffers hold paths * span
 * tokens); a record whose path or length lies outside it commits nothing.
 * ------------------------------------------------------------------------ */
#define VMI_TREE_ATTENTION 1
#define VMI_TREE_GDN 2
typedef struct vmi_tree_layer {
    int kind;                          /* VMI_TREE_ATTENTION or VMI_TREE_GDN */
    int n_kv_heads, max_len;           /* attention */
    int n_k_heads, n_v_heads, n_slots; /* Gated DeltaNet */
    uint16_t* k_cache;                 /* attention: the layer's caches and tree_kv */
    uint16_t* v_cache;
    const uint16_t* tree_kv;
    uint16_t* conv_ring;               /* Gated DeltaNet: the rings, tree_conv and tree_side */
    float* state_ring;
    const uint16_t* tree_conv;
    const float* tree_side;
} vmi_tree_layer;

size_t vmi_attention_tree_workspace_bytes(int paths, int span, int hidden, int n_heads, int n_kv_heads, int max_len);
int vmi_attention_tree(const vmi_attn_layer_desc* desc, const uint16_t* x, int paths, int span, int pos0,
                       const int32_t* pos_device, const uint16_t* k_cache, const uint16_t* v_cache, int max_len,
                       uint16_t* tree_kv, uint16_t* out, void* workspace, size_t workspace_bytes, void* stream);
int vmi_gdn_tree(const vmi_gdn_layer_desc* desc, const uint16_t* x, int paths, int span, int pos0,
                 const int32_t* pos_device, const uint16_t* conv_ring, const float* state_ring, int n_slots,
                 uint16_t* tree_conv, float* tree_side, uint16_t* out, void* workspace, size_t workspace_bytes,
                 void* stream);
int vmi_tree_commit(const int32_t* result, const vmi_tree_layer* layers, int n_layers, int max_heads, int paths,
                    int span, int pos0, const int32_t* pos_device, void* stream);

/* ------------------------------------------------------------------------
 * vmi_rmsnorm -- out = bf16(x * 1/sqrt(mean(x^2) + eps) * weight) per token
 * (mlx RMSNorm as the MTP module applies it: pre_fc_norm_embedding,
 * pre_fc_norm_hidden and norm, qwen3_next_mtp.py:27-31, 46-49, 54).  With ids
 * (int32 [T]) the rows are gathered from the table x [rows, hidden] first -
 * the embedding lookup embed_tokens(next_ids) of qwen3_next_mtp.py:46; an id
 * outside [0, rows) reads row 0 and sets VMI_STATUS_BAD_SLOT in *status
 * (may be NULL).  weight NULL: the rows are copied unnormalised (the main
 * model's embedding lookup).  Output row t starts at out + t * out_stride
 * (out_stride >= hidden: writes one half of a concatenation in place).
 * hidden a multiple of 512; x, weight, out 16-byte aligned.
 * ------------------------------------------------------------------------ */
int vmi_rmsnorm(const uint16_t* x, const int32_t* ids, int rows, int T, int hidden, const uint16_t* weight, float eps,
                uint16_t* out, int out_stride, uint32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * vmi_topk_rows -- the k largest entries of each row of f32 logits
 * [rows, vocab] in descending order (ties to the lower index, NaN last): the
 * drafter's top-P first tokens of draft_paths (mlx_streaming/mtp/drafter.py:
 * 150-160, mx.argsort(lg)[-P:][::-1]).  ids int32 [rows, k]; vals f32
 * [rows, k] or NULL.  k <= 16.
 * ------------------------------------------------------------------------ */
int vmi_topk_rows(const float* logits, int rows, int vocab, int k, int32_t* ids, float* vals, void* stream);

/* ------------------------------------------------------------------------
 * Acceptance.  Every entry point writes an int32 result record of 4 + K + 1
 * entries: [0] n_emitted, [1] matched (drafts accepted), [2] accepted_len
 * (verify positions whose state is kept), [3] winning path (-1: no finite
 * logit in some row, nothing emitted), [4 ..] the emitted tokens.
 *
 * vmi_accept_greedy -- replaces accept_prefix and the emission rules
 *   mlx_streaming/mtp/generate.py:338-351 (longest prefix with preds == drafts),
 *   :819 (accepted_len = min(matched + 1, K)), :850-856 (drafts[:m] + [preds[m]],
 *   or drafts[:K] when all match), and tree_verify_step's winner selection
 *   :379-386 (most matches, ties to the lower path index).
 * drafts int32 [P, K]; preds int32 [P, K + mode] (argmax of the verify
 * logits, e.g. from vmi_lm_head).  mode 0: the verify batch is [x, d1..d_{K-1}]
 * (the reference's T = K layout, K predictions); mode 1: [x, d1..dK] (T = K+1,
 * emits drafts[:m] + [preds[m]] for every m <= K, accepted_len = m + 1; P = 1).
 * K <= 15, P <= 65535.
 * ------------------------------------------------------------------------ */
int vmi_accept_greedy(const int32_t* drafts, const int32_t* preds, int P, int K, int mode, int32_t* result,
                      void* stream);

/* ------------------------------------------------------------------------
 * vmi_spec_commit -- the commit of one speculative step on the device, after
 * vmi_accept_greedy, so that a captured step needs no host round trip.  With
 * acc = accepted_len and w = the winning path of the record:
 *   H = hid[w][acc - 1] (bf16 [hidden]; hid [paths][rows][hidden] holds the
 *   pre-norm hidden of the verify rows), x = the last emitted token,
 *   pos += acc, mtp_len += acc, mtp_pos[i] = mtp_len + i for i < K (the next
 *   step's draft positions).
 * Both verify layouts: rows = K + 1 after a mode-1 record (T = K + 1, acc =
 * matched + 1, a bonus token when every draft matches), rows = the step's
 * verify length after a mode-0 record (the reference's T = K layout: acc =
 * min(matched + 1, rows), x = the last draft when all match), paths > 1 for
 * a tree.  Replaces the state update of the reference's decode loop:
 * mlx_streaming/mtp/generate.py:819 (accepted_len), :850-856 (new tokens and
 * the next input x), :895 (H_last = rH[:, -1]) and kv_cache.py:222-251
 * (committing the accepted prefix by setting lengths); tree_verify_step's
 * winner row, generate.py:386 and :416-420.  A record with no emitted token, acc
 * outside [1, rows], more than rows tokens or a path outside [0, paths)
 * changes nothing and ORs VMI_STATUS_BAD_RECORD into *status (may be NULL).
 * H must not overlap hid.  K <= 15, rows <= 16.
 * ------------------------------------------------------------------------ */
int vmi_spec_commit(const int32_t* result, const uint16_t* hid, int rows, int paths, int hidden, int K, uint16_t* H,
                    int32_t* x, int32_t* pos, int32_t* mtp_len, int32_t* mtp_pos, uint32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * vmi_accept_stochastic -- speculative sampling (Leviathan et al. 2023,
 * Algorithm 1; Chen et al. 2023) in one kernel.  No reference counterpart:
 * the reference accepts greedily only (generate.py:338-351); this is the
 * published method on its verify layout.
 * target_logits f32 [K+1, vocab] (verify rows of [x, d1..dK]); draft_logits
 * f32 [K, vocab] (the drafter's rows that d1..dK were sampled from) or NULL
 * for greedy drafts (q one-hot at each draft); drafts int32 [K].
 * p, q = temperature / top-p transforms on integer masses:
 *   W_j = floor(2^31 * 2^((l_j - max l) * s)), s = fp32((1/temperature)*log2 e),
 *   nucleus = {W_j >= theta}, theta the largest value whose at-or-above mass
 *   reaches ceil(top_p * sum W) (ties join together), p(j) = W_j / nucleus mass.
 * Draft i is kept when U_i 2^-32 * q(d_i) <= p(d_i) and p(d_i) > 0; at the first
 * rejection the token is drawn from floor(2^31 max(0, p - q)) masses (from p
 * when those are all zero); with every draft kept a bonus token is drawn from
 * p_K.  Draws: t = floor(V_i * total / 2^32), token = first index whose
 * running mass exceeds t.  (U_i, V_i) = words 0, 1 of Philox4x32-10 with key
 * seed and counter (offset lo, offset hi, i, 0x5A3D1E57).  Bit-identical to
 * the CPU oracle.  temperature > 0 (use vmi_accept_greedy for 0), 0 < top_p <= 1.
 * offset_device (uint64 on the device, or NULL): when set, the counter
 * offset is offset + *offset_device, read when the kernel runs (a captured
 * graph replays with offsets that advance on the device).
 * workspace: vmi_accept_stochastic_workspace_bytes(K, vocab, draft_logits != NULL)
 * bytes, zero before the first call and left so by every call; one call in
 * flight per workspace.  The kernel's workgroups wait for each other between
 * its phases, so all of them must be resident at once (the grid holds at
 * most min(2, the occupancy calculator's figure) workgroups per CU); a wait
 * that outlasts its bound (the CUs held by other work; vmi_set_wait_limit)
 * gives up, and the call then writes record [0, 0, 0, -1] and ORs
 * VMI_STATUS_WAIT_GAVE_UP into *status; a logit row with no finite value
 * writes the same record and ORs VMI_STATUS_BAD_LOGITS.  status (uint32 on
 * the device, or NULL) is the caller's: the kernel never clears it.
 * ------------------------------------------------------------------------ */
size_t vmi_accept_stochastic_workspace_bytes(int K, int vocab, int has_draft_logits);
int vmi_accept_stochastic(const float* target_logits, const float* draft_logits, const int32_t* drafts, int K,
                          int vocab, float temperature, float top_p, uint64_t seed, uint64_t offset,
                          const uint64_t* offset_device, int32_t* result, void* workspace, size_t workspace_bytes,
                          uint32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * vmi_sample_top_p -- one token per row of logits f32 [rows, vocab] from the
 * same temperature / top-p distribution (row r uses V_r of counter
 * (offset, r)); the drafter's sampler when drafting stochastically.  The
 * reference drafts by argmax only (drafter.py:20-40).  out int32 [rows]
 * (-1 for a row without a finite logit, and for a row drawn after one of the
 * kernel's waits outlasted its bound; the status bits as for
 * vmi_accept_stochastic).  offset_device, workspace, residency and status as
 * for vmi_accept_stochastic.
 * ------------------------------------------------------------------------ */
size_t vmi_sample_top_p_workspace_bytes(int rows, int vocab);
int vmi_sample_top_p(const float* logits, int rows, int vocab, float temperature, float top_p, uint64_t seed,
                     uint64_t offset, const uint64_t* offset_device, int32_t* out, void* workspace,
                     size_t workspace_bytes, uint32_t* status, void* stream);

/* ------------------------------------------------------------------------
 * vmi_set_wait_limit -- the bound (in polls: a coherent load and a short sleep) of the
 * co-residency waits of vmi_accept_stochastic and vmi_sample_top_p, for
 * calls launched afterwards from any thread; polls <= 0 restores the
 * default (65,536).  Returns the previous bound.  No reference counterpart:
 * tests force the give-up path with a bound of 1, so the kernels still exit
 * normally.
 * ------------------------------------------------------------------------ */
int vmi_set_wait_limit(int polls);

/* ------------------------------------------------------------------------
 * Synthetic data (no reference counterpart: the reference loads real
 * checkpoints).  Bit-identical to the CPU generator used by the tests:
 * element i = (sum of four 16-bit words of Philox4x32-10 block i/2 -
 * 131070) * scale, quantised per group of 64 by min/max with bf16
 * scale/bias.  vmi_synth_quantized fills a [rows, cols] projection;
 * vmi_synth_bf16 fills n bf16 values.
 * ------------------------------------------------------------------------ */
int vmi_synth_quantized(uint64_t seed, uint32_t stream_id, int64_t rows, int cols, int group, int bits, float scale,
                        uint32_t* w, uint16_t* s, uint16_t* b, void* stream);
int vmi_synth_bf16(uint64_t seed, uint32_t stream_id, int64_t n, float scale, uint16_t* out, void* stream);

/* ------------------------------------------------------------------------
 * Device ceilings (no reference counterpart: the reference publishes no
 * kernel figures).  Measurement kernels whose rates are the denominators a
 * benchmark reports beside the published peaks.
 * vmi_stream_read reads bytes at src once with 16-byte loads (nontemporal
 * loads when nontemporal != 0), `workgroups` workgroups of 256 lanes each
 * striding over 32 KB chunks; workgroup g stores the XOR of the 32-bit words
 * it read to sink[g] (uint32 [workgroups]), so the XOR of sink is the XOR of
 * the whole buffer.  src 16-byte aligned, bytes a non-zero multiple of 16.
 * vmi_mfma_peak runs `workgroups` workgroups of four waves; each wave issues
 * iters rounds of four independent v_mfma_f32_16x16x32_f16 of 16,384 flops
 * each (16 * iters * 16,384 dense flops per workgroup), and workgroup g
 * writes to sink[g] (float [workgroups]) the sum of element 0..3 of its first
 * lane's four accumulators (chain j's element j).
 * ------------------------------------------------------------------------ */
int vmi_stream_read(const void* src, size_t bytes, int nontemporal, int workgroups, uint32_t* sink, void* stream);
int vmi_mfma_peak(int workgroups, int iters, float* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VMI_H_ */
