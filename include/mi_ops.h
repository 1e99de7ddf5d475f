/*
 * mi_ops.h -- C ABI of the MI355X (gfx950) per-layer fused ops.
 *
 * Each entry point takes ggml-style tensor views (ne[0] innermost, byte
 * strides nb[]) and reproduces the ggml op, or the chain of ggml ops, that
 * acestep.cpp's graph builders emit at that point of the graph, so host code
 * can call it at the same graph boundary. All calls are asynchronous and
 * stream-ordered on the given HIP stream (NULL = the null stream). The
 * library never allocates, frees or retains caller memory; arguments are
 * validated on the host before any launch, and no entry point aborts: a
 * non-zero mi_status is returned instead.
 *
 * Types: MI_TYPE_* values equal the matching enum ggml_type values, so a
 * ggml backend can pass tensor->type, tensor->ne and tensor->nb through.
 *
 * Q8_0 tensors follow ggml: ne[0] counts elements (a multiple of 32), nb[0]
 * is the 34-byte block size, a block is { fp16 d; int8 qs[32] }.
 *
 * Activation tensors may be F32 or BF16 (BF16 is computed as bf16 -> f32,
 * the fp32 op chain, f32 -> bf16 round-to-nearest-even at the output).
 * Norm weights and AdaLN vectors are F32, as the reference stores them.
 */
#ifndef MI_OPS_H
#define MI_OPS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_OPS_ABI_VERSION 2

enum mi_type {
    MI_TYPE_F32  = 0,
    MI_TYPE_F16  = 1,
    MI_TYPE_Q8_0 = 8,
    MI_TYPE_I32  = 26,
    MI_TYPE_BF16 = 30,
};

enum mi_status {
    MI_OK              = 0,
    MI_ERR_NULL        = -1, /* a required tensor or data pointer is NULL        */
    MI_ERR_TYPE        = -2, /* unsupported type or type combination             */
    MI_ERR_SHAPE       = -3, /* shapes are inconsistent for the op               */
    MI_ERR_STRIDE      = -4, /* unsupported stride (e.g. nb[0] != element size)  */
    MI_ERR_ALIGN       = -5, /* data pointer or stride misaligned for its type   */
    MI_ERR_PARAM       = -6, /* invalid scalar parameter                         */
    MI_ERR_UNSUPPORTED = -7, /* valid ggml op configuration this library lacks   */
    MI_ERR_HIP         = -8, /* the HIP runtime reported an error at launch      */
    MI_ERR_FILE        = -9, /* a file is missing, unreadable, truncated or not GGUF */
    MI_ERR_SCRATCH     = -10, /* the call needs more than the library's static scratch */
};

/* Q8_0 quantizer rounding variants (both are ggml's own):
 *   MI_Q8_0_CPU_X86: ggml-cpu x86 from_float: id = 127/amax, round half to even
 *   MI_Q8_0_REF:     quantize_row_q8_0_ref:  id = 1/(amax/127), roundf (half away) */
enum mi_q8_0_rounding {
    MI_Q8_0_CPU_X86 = 0,
    MI_Q8_0_REF     = 1,
};

typedef struct mi_tensor {
    void *   data;
    int32_t  type;     /* enum mi_type */
    int32_t  reserved; /* must be 0 */
    int64_t  ne[4];    /* elements per dimension, ne[0] innermost */
    uint64_t nb[4];    /* byte strides */
} mi_tensor;

typedef void * mi_stream; /* hipStream_t */

int          mi_abi_version(void);
const char * mi_status_str(int status);

/* ggml_rms_norm(x, eps), followed by ggml_mul(., w) when w != NULL.
 * Replaces qwen3_rms_norm (qwen3-enc.h:114-120; called at qwen3-lm.h:471,
 * 485, 494, 632, 736, 745), dit_ggml_rms_norm_weighted (dit-graph.h:24-30;
 * 429 cross-attn norm) and the QK-norm without rope of the DiT cross
 * attention (dit-graph.h:328-331).
 * x, y: [n, ...] F32/BF16, rows may be strided (nb[0] = element size);
 * w: F32 [n] or NULL. Reduction: float squares summed in double for F32
 * rows (ggml-cpu's order of operations), in fp32 for BF16 rows;
 * mean = sum/n, scale = 1.0f/sqrtf(mean + eps). */
int mi_rms_norm(const mi_tensor * x, const mi_tensor * w, float eps, const mi_tensor * y, mi_stream stream);

/* RMSNorm * w then AdaLN modulate, fused:
 * y = ((rms_norm(x) * w) * (scale + 1)) + shift.
 * Replaces dit_ggml_rms_norm_weighted + dit_ggml_adaln (dit-graph.h:404-405,
 * 442-443, 605-606; adaln at 54-64). scale, shift: F32 [n]. */
int mi_rms_norm_modulate(const mi_tensor * x, const mi_tensor * w, const mi_tensor * scale, const mi_tensor * shift,
                         float eps, const mi_tensor * y, mi_stream stream);

/* Residual add fused with the RMSNorm that consumes it:
 *   y_sum  = residual + x            (gate == NULL; ggml_add)
 *          = residual + x * gate     (dit_ggml_gated_add, dit-graph.h:70-76)
 *   y_sum  = clamp(y_sum, lo, hi)    when clamp != 0 (ggml_clamp)
 *   y_norm = rms_norm(y_sum) [* w] [* (scale + 1) + shift]
 * Replaces, in one pass over the activations, the add -> norm node pairs at
 * dit-graph.h:420 -> 429/442-443, dit-graph.h:432 -> 442-443 and
 * qwen3-lm.h:730-736 (residual add + clamp -> post-attention norm),
 * 738-741 -> 632 of the next layer. y_sum is stored in the activation type
 * and y_norm is computed from that stored value, so the results equal the
 * unfused kernels'. All four activations share one type and shape; y_sum may
 * alias residual; y_norm must not alias any input or y_sum. scale/shift need
 * w (as dit_ggml_adaln follows dit_ggml_rms_norm_weighted). */
int mi_add_rms_norm(const mi_tensor * residual, const mi_tensor * x, const mi_tensor * gate, int clamp, float lo,
                    float hi, const mi_tensor * w, const mi_tensor * scale, const mi_tensor * shift, float eps,
                    const mi_tensor * y_sum, const mi_tensor * y_norm, mi_stream stream);

/* ggml_rope_ext(x, pos, NULL, n_dims, mode, n_ctx_orig=0, freq_base, freq_scale,
 * ext_factor, attn_factor, beta_fast, beta_slow) for mode 2 (NEOX).
 * Replaces the rope nodes at qwen3-enc.h:173-174, qwen3-lm.h:378-379,
 * 666-667, dit-graph.h:194-196. x, y: [ne0, heads, n_pos, ne3] F32/BF16,
 * pos: I32 [n_pos] (one position per ne2 index, reused across ne3).
 * Supported: mode == 2, ext_factor == 0 (the only values the reference
 * passes), n_dims even and <= ne0 (remaining dims are copied). */
int mi_rope_ext(const mi_tensor * x, const mi_tensor * pos, int n_dims, int mode, float freq_base, float freq_scale,
                float ext_factor, float attn_factor, const mi_tensor * y, mi_stream stream);

/* Per-head QK-RMSNorm then NEOX rope for Q and K in one launch:
 *   q_out = rope(rms_norm(q) * q_w),  k_out = rope(rms_norm(k) * k_w)
 * Replaces rms_norm + mul + rope (x2) at qwen3-lm.h:372-379, 660-667,
 * qwen3-enc.h:165-174, dit-graph.h:183-196. q/k may be strided views of the
 * fused QKV projection output (the ggml_cont copies at qwen3-lm.h:640-642,
 * dit-graph.h:160-163 are not needed). k/k_w/k_out may be NULL (Q only);
 * q_w/k_w NULL means no norm (plain rope). Same head size for q and k. */
int mi_qk_norm_rope(const mi_tensor * q, const mi_tensor * q_w, const mi_tensor * q_out, const mi_tensor * k,
                    const mi_tensor * k_w, const mi_tensor * k_out, const mi_tensor * pos, float eps, int n_dims,
                    float freq_base, float freq_scale, float attn_factor, mi_stream stream);

/* ggml_swiglu(gu) / ggml_glu(gu, SWIGLU, swapped): gu [2n, rows] -> y [n, rows],
 * y = silu(gate) * up, gate = first half of ne0 (second half if swapped).
 * Replaces qwen3-enc.h:217, dit-graph.h:259. */
int mi_swiglu(const mi_tensor * gu, int swapped, const mi_tensor * y, mi_stream stream);

/* ggml_swiglu_split(g, u): y = silu(g) * u. Replaces qwen3-enc.h:221,
 * dit-graph.h:264. */
int mi_swiglu_split(const mi_tensor * g, const mi_tensor * u, const mi_tensor * y, mi_stream stream);

/* ggml_add(a, b): b same shape as a, or F32 [ne0] broadcast over rows, or
 * any ggml_can_repeat(b, a) shape (slower path). Replaces the residual adds
 * at qwen3-enc.h:238, 243, qwen3-lm.h:479, 487, 730, 738, dit-graph.h:432
 * and the AdaLN vector build at dit-graph.h:391. */
int mi_add(const mi_tensor * a, const mi_tensor * b, const mi_tensor * y, mi_stream stream);

/* ggml_mul(a, b), same broadcast rules as mi_add. */
int mi_mul(const mi_tensor * a, const mi_tensor * b, const mi_tensor * y, mi_stream stream);

/* ggml_clamp(ggml_add(a, b), lo, hi); b may be NULL (clamp only).
 * Replaces qwen3-lm.h:479-482, 487-490, 730-733, 738-741 and the V clamp at
 * qwen3-lm.h:393, 676. */
int mi_add_clamp(const mi_tensor * a, const mi_tensor * b, float lo, float hi, const mi_tensor * y,
                 mi_stream stream);

/* dit_ggml_gated_add (dit-graph.h:70-76): y = residual + (x * gate),
 * gate F32 [ne0] (raw, no sigmoid). Used at dit-graph.h:420, 445. */
int mi_gated_add(const mi_tensor * residual, const mi_tensor * x, const mi_tensor * gate, const mi_tensor * y,
                 mi_stream stream);

/* dit_ggml_adaln (dit-graph.h:54-64) alone: y = (x * (scale + 1)) + shift. */
int mi_modulate(const mi_tensor * x, const mi_tensor * scale, const mi_tensor * shift, const mi_tensor * y,
                mi_stream stream);

/* ggml_get_rows(table, ids): table [n, n_rows] Q8_0/F16/BF16/F32, ids I32
 * [n_ids] -> y [n, n_ids] F32 (or BF16). Replaces the embedding lookups at
 * qwen3-enc.h:390, 465, qwen3-lm.h:464, 626. ids may be strided (nb[0] any
 * multiple of 4, as ggml reads src1 through nb10). An id outside [0, n_rows)
 * yields a zero row and, when d_err != NULL, increments *d_err (device
 * int32) -- ggml-cpu aborts there instead. */
int mi_get_rows(const mi_tensor * table, const mi_tensor * ids, const mi_tensor * y, int32_t * d_err,
                mi_stream stream);

/* ggml_cpy(src, dst): src F32/BF16/F16, dst F32/BF16/F16/Q8_0 view of the
 * same shape (any strides; Q8_0 dst rows are whole blocks). Q8_0 uses the
 * ggml-cpu x86 from_float rounding (MI_Q8_0_CPU_X86). Replaces the KV-cache
 * writes at qwen3-lm.h:405-406, 701-702, songgen-lelm-gen.h:264-265,
 * 559-560. */
int mi_cpy(const mi_tensor * src, const mi_tensor * dst, mi_stream stream);

/* mi_cpy with an explicit Q8_0 rounding variant (enum mi_q8_0_rounding). */
int mi_cpy_q8_0(const mi_tensor * src, const mi_tensor * dst, int rounding, mi_stream stream);

/* KV-cache store for a batch of sequences in one launch, replacing the N
 * per-sequence ggml_cpy nodes per layer of qw3lm_forward_batch
 * (qwen3-lm.h:682-703) and the prefill cpy (qwen3-lm.h:396-406,
 * songgen-lelm-gen.h:254-265, 548-562).
 *   k, v:       [D, Nkv, T, B]  F32/BF16/F16 (v may be NULL)
 *   k/v_cache:  [D, max_seq, Nkv, n_sets] Q8_0/F16/BF16/F32
 *   pos0:       I32 [B]   first slot written for sequence b
 *   sets:       I32 [B] or NULL (set = b)
 * cache[:, pos0[b] + t, h, sets[b]] = k[:, h, t, b]. Out-of-range slots or
 * sets are skipped and counted in *d_err when d_err != NULL. */
int mi_kv_store(const mi_tensor * k, const mi_tensor * k_cache, const mi_tensor * v, const mi_tensor * v_cache,
                const mi_tensor * pos0, const mi_tensor * sets, int rounding, int32_t * d_err, mi_stream stream);

/* QK-norm -> NEOX rope and the KV-cache store as one launch, replacing a
 * decode step's q/k norms, ropes, V clamp and per-sequence ggml_cpy nodes
 * (qwen3-lm.h:660-703). Equal, bit for bit, to mi_qk_norm_rope(q, q_w, q_out,
 * k, k_w, k_out, pos, ...), then (clamp_v) mi_add_clamp(v, NULL, -65504,
 * 65504, v), then mi_kv_store of k_out and v viewed as B = pos0.ne[0]
 * sequences of tokens / B tokens each (token t of the flat ne2 * ne3 order is
 * token t % T of sequence t / T): the roped K never goes to memory and V is
 * not modified.
 *   q, q_out: [D, Nh, ne2, ne3]; k, v: [D, Nkv, ne2, ne3]; one activation type
 *   q_w, k_w: F32 [D] or both NULL (rope only); pos: I32 [ne2]
 *   k_cache, v_cache: [D, max_seq, Nkv, n_sets], one type (Q8_0/F16/BF16/F32)
 *   pos0, sets, rounding, d_err: as mi_kv_store
 * Needs D in {64, 128, 256} rotated whole (n_dims == D) and 16-byte aligned
 * q/k/v/q_out rows (2-byte for Q8_0 caches, 16-byte otherwise); other
 * layouts return MI_ERR_UNSUPPORTED (use the three calls). */
int mi_qk_norm_rope_kv_store(const mi_tensor * q, const mi_tensor * q_w, const mi_tensor * q_out, const mi_tensor * k,
                             const mi_tensor * k_w, const mi_tensor * v, const mi_tensor * pos, float eps, int n_dims,
                             float freq_base, float freq_scale, float attn_factor, int clamp_v,
                             const mi_tensor * k_cache, const mi_tensor * v_cache, const mi_tensor * pos0,
                             const mi_tensor * sets, int rounding, int32_t * d_err, mi_stream stream);

/* ggml_scale(x, s): y = x * s, one fp32 multiply per element (the result
 * rounded to y's type). Replaces the timestep scaling ggml_scale(t, 1000) in
 * front of the embedding (dit-graph.h:87). x, y: activations of one shape
 * (F32/BF16/F16, contiguous rows, any row strides); y == x allowed. */
int mi_scale(const mi_tensor * x, float s, const mi_tensor * y, mi_stream stream);

/* ggml_timestep_embedding(t, dim, max_period): t F32 [n] -> y F32 [dim, n].
 * Replaces dit-graph.h:90 (dim 256, max_period 10000). */
int mi_timestep_embedding(const mi_tensor * t, int dim, int max_period, const mi_tensor * y, mi_stream stream);

/* ggml_flash_attn_ext(q, k, v, mask, scale, max_bias, logit_softcap) with
 * GGML_PREC_F32. Replaces the DiT self and cross attention
 * (dit-graph.h:227-231, 348-349), the LM prefill attention over the KV cache
 * (qwen3-lm.h:414-417; songgen-lelm-gen.h:276-277, F16 or Q8_0 cache) and the
 * batched decode attention over it (qwen3-lm.h:718-723, 256-bucketed read
 * length at 582-596; songgen-lelm-gen.h:582-583).
 *   q:    [D, n_q, Nh, N]      F32/BF16/F16
 *   k, v: [D, n_kv, Nkv, Nk3]  both F16, both BF16, both Q8_0 or both F32
 *         (F32 only for D <= 128); Nh % Nkv == 0, N % Nk3 == 0; rows at a
 *         16-byte aligned stride (Q8_0: 8-byte when D % 128 == 0, else
 *         4-byte), e.g. cache views
 *   mask: F16 [n_kv, >= n_q, mne2, mne3] (head h uses h % mne2, batch b uses
 *         b % mne3) or NULL
 *   y:    F32 [D, Nh, n_q, N]  (ggml's permuted result)
 * D (= ne0 of q, k and v) is 64, 128 or 256. max_bias and logit_softcap must
 * be 0 (the only values the reference passes); others return
 * MI_ERR_UNSUPPORTED. q is converted to K's dot type as ggml-cpu converts it
 * (fp16, bf16, or Q8_0 with the x86 rounding); keys whose mask is -inf do not
 * contribute; a row whose keys are all masked is NaN. The decode and split
 * kernels never read masked keys; the matrix-core prefill kernel (64 or more
 * (query, head) rows per KV head, D = 128) reads the K/V rows of keys masked
 * for only some rows of a 64-key tile and multiplies them by 0, so F16/BF16
 * rows there must be finite (the reference clears its caches at allocation);
 * a Q8_0 V block with a non-finite scale counts as 0.
 * workspace: device memory of at least mi_flash_attn_ext_workspace() bytes
 * (for the partial results of a split key range; NULL when that is 0). The
 * size depends on the shapes and on the current device's CU count. */
int mi_flash_attn_ext_workspace(const mi_tensor * q, const mi_tensor * k, const mi_tensor * v, size_t * bytes);
int mi_flash_attn_ext(const mi_tensor * q, const mi_tensor * k, const mi_tensor * v, const mi_tensor * mask,
                      float scale, float max_bias, float logit_softcap, const mi_tensor * y, void * workspace,
                      size_t workspace_bytes, mi_stream stream);

/* ggml_mul_mat(w, x) with Q8_0 weights, as ggml-cpu computes it: each row of x
 * is quantized to Q8_0 with the x86 from_float (id = 127 / amax, round to
 * nearest even, saturate) and each output is sum_b (d_w * d_x) * sum_i q_w q_x
 * with an exact int32 dot per 32-block, accumulated in fp32
 * (ggml_vec_dot_q8_0_q8_0). Replaces the Q8_0 linear layers qwen3_linear
 * (qwen3-enc.h:86-88; called at qwen3-lm.h:639-651, 729, 737 via
 * qwen3-enc.h:216-223) and dit_ggml_linear (dit-graph.h:36-49), and the LM head
 * over the Q8_0 token table (qwen3-lm.h:755).
 * Weights are repacked once, at load (as ggml-cpu's repacking buffer types
 * do): mi_q8_0_repack copies a Q8_0 [k, n] weight (GGUF layout, rows at
 * stride nb[1]) into dst, a lossless layout of mi_q8_0_repack_bytes(k, n)
 * bytes (rows in groups of 64; 34 bytes per block).
 * mi_mul_mat_q8_0: w = repacked weight [k, n]; x F32 [k, m] (m = ne1 * ne2 *
 * ne3 rows, uniformly strided; up to 8 rows take the matrix-vector kernel,
 * more the matrix-core kernel); y F32 [n, m]. workspace: device memory of at
 * least mi_mul_mat_q8_0_workspace() bytes, 256-byte aligned (the quantized x,
 * and the partial sums of a split k). Calls sharing a workspace race. */
int mi_q8_0_repack_bytes(int64_t k, int64_t n, size_t * bytes);
int mi_q8_0_repack(const mi_tensor * w, void * dst, size_t dst_bytes, mi_stream stream);
int mi_mul_mat_q8_0_workspace(int64_t k, int64_t n, const mi_tensor * x, size_t * bytes);
int mi_mul_mat_q8_0(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * y,
                    void * workspace, size_t workspace_bytes, mi_stream stream);

/* mi_mul_mat_q8_0 without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Its scratch (the quantized x and the partial sums of
 * a split k) is one static device array of MI_MUL_MAT_NOALLOC_SCRATCH_BYTES
 * per GPU, held until the process ends; a call that needs more
 * (mi_mul_mat_q8_0_workspace() above the limit: Qwen3 decode at any batch up
 * to 8 and prefill chunks up to about m * k = 28M fit) returns MI_ERR_SCRATCH
 * before any launch. Every call on one GPU uses the same array, so calls that
 * overlap on one GPU (other streams, other host threads) race; stream-ordered
 * calls do not. Nothing in it has to start at zero: every scratch value that
 * feeds a stored y element is written by the same call. (The matrix kernel,
 * m > 8, reads the quantized x of the padding rows m .. 128*ceil(m/128)-1,
 * which an earlier call may have left there; those rows only produce y rows
 * that are never stored.) y is bit-identical to mi_mul_mat_q8_0's. */
#define MI_MUL_MAT_NOALLOC_SCRATCH_BYTES ((size_t) 32 << 20)
int mi_mul_mat_q8_0_noalloc(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * y,
                            mi_stream stream);

/* The SwiGLU -> down projection pair as one call: y = ggml_mul_mat(w,
 * ggml_swiglu(gu)) (qwen3-enc.h:221-223, the Qwen3 MLP; dit-graph.h:265-268,
 * the DiT MLP). gu F32 [2k, m] (gate = first half of each row, or the second
 * when swapped), w repacked [k, n], y F32 [n, m]. The SwiGLU values are
 * computed inside the quantization of x, with the arithmetic of mi_swiglu, so
 * y is bit-identical to mi_swiglu followed by mi_mul_mat_q8_0; the [k, m]
 * SwiGLU output never goes to memory. Workspace as mi_mul_mat_q8_0 for an x
 * of m rows of k. */
int mi_mul_mat_q8_0_swiglu_workspace(int64_t k, int64_t n, const mi_tensor * gu, size_t * bytes);
int mi_mul_mat_q8_0_swiglu(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped,
                           const mi_tensor * y, void * workspace, size_t workspace_bytes, mi_stream stream);

/* The down projection with the residual add after it, as one call:
 * y = ggml_add(ggml_mul_mat(w, ggml_swiglu(gu)), r), then ggml_clamp(y, lo, hi)
 * when clamp != 0 (qwen3-lm.h:736-741: the MLP output added to the
 * post-attention residual, clamped to the fp16 range under clamp_fp16). r F32
 * of y's shape (rows uniformly strided; y may be r). The residual is added
 * where the product's sum is formed, so y is bit-identical to
 * mi_mul_mat_q8_0_swiglu followed by mi_add (or mi_add_clamp), without the
 * product's round trip through memory or the extra launch. Workspace as
 * mi_mul_mat_q8_0_swiglu. */
int mi_mul_mat_q8_0_swiglu_add(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped,
                               const mi_tensor * r, int clamp, float lo, float hi, const mi_tensor * y, void * workspace,
                               size_t workspace_bytes, mi_stream stream);

/* The DiT's MLP tail as one call: y = r + ggml_mul_mat(w, ggml_swiglu(gu)) *
 * gate (dit_ggml_gated_add after dit_ggml_build_mlp, dit-graph.h:439-440, 68-76:
 * the product multiplied by the F32 [n] gate vector, rounded, then added to r),
 * bit-identical to mi_mul_mat_q8_0_swiglu followed by mi_gated_add. Operands and
 * workspace as mi_mul_mat_q8_0_swiglu_add (without the clamp); y may be r. */
int mi_mul_mat_q8_0_swiglu_gated_add(const void * w, int64_t k, int64_t n, const mi_tensor * gu, int swapped,
                                     const mi_tensor * r, const mi_tensor * gate, const mi_tensor * y, void * workspace,
                                     size_t workspace_bytes, mi_stream stream);

/* The RMSNorm -> product pair as one call: y = ggml_mul_mat(w,
 * ggml_mul(ggml_rms_norm(x, eps), norm_w)) (qwen3-lm.h:632-639, the input norm
 * feeding the fused QKV projection; qwen3_rms_norm, qwen3-enc.h:114-120). x F32
 * [k, m], norm_w F32 [k], y F32 [n, m]. The normalized rows are computed inside
 * the quantization of x with the arithmetic of mi_rms_norm (only the order of
 * the double additions of the sum of squares differs), so y equals
 * mi_rms_norm followed by mi_mul_mat_q8_0 and the normalized rows never go to
 * memory. Workspace: mi_mul_mat_q8_0_workspace() for the same x. */
int mi_mul_mat_q8_0_rms_norm(const void * w, int64_t k, int64_t n, const mi_tensor * x, const mi_tensor * norm_w,
                             float eps, const mi_tensor * y, void * workspace, size_t workspace_bytes,
                             mi_stream stream);

/* The same with the residual add before the norm: sum = a + b (written, F32 [k,
 * m], for the next residual), y = ggml_mul_mat(w, rms_norm(sum) * norm_w)
 * (qwen3-lm.h:729-737: the attention residual, the post-attention norm and the
 * gate/up projection), equal to mi_add_rms_norm followed by mi_mul_mat_q8_0.
 * a, b, sum: F32 [k, m], uniformly strided rows; sum must not overlap a or b
 * (MI_ERR_PARAM). Workspace as mi_mul_mat_q8_0 for x = a. */
int mi_mul_mat_q8_0_add_rms_norm(const void * w, int64_t k, int64_t n, const mi_tensor * a, const mi_tensor * b,
                                 const mi_tensor * norm_w, float eps, const mi_tensor * sum, const mi_tensor * y,
                                 void * workspace, size_t workspace_bytes, mi_stream stream);

/* The DiT's norm -> product pairs as one call (dit_ggml_build_layer,
 * dit-graph.h:402-439): the optional residual add before the norm, gated or
 * plain (sum = a + b * gate, or a + b; written to sum, F32 [k, m], for the next
 * residual), the RMSNorm * norm_w, the optional AdaLN modulate
 * ((x' * (scale + 1)) + shift, dit_ggml_adaln, dit-graph.h:54-64), then
 * y = ggml_mul_mat(w, x'). Replaces the node chains feeding the QKV projection
 * (404-405, norm -> modulate), the cross-attention Q projection (415 and 424,
 * gated add -> norm) and the gate/up projection (415 or 427, then 437-438,
 * add -> norm -> modulate). b, gate and sum may be null (no add; gate needs b);
 * scale and shift are both given or both null; gate, norm_w, scale, shift:
 * F32 [k]. Every step is rounded as mi_add_rms_norm / mi_rms_norm_modulate round
 * it, so y equals that call followed by mi_mul_mat_q8_0 and the normalized rows
 * never go to memory. Same operand rules and workspace as
 * mi_mul_mat_q8_0_add_rms_norm. */
int mi_mul_mat_q8_0_adaln(const void * w, int64_t k, int64_t n, const mi_tensor * a, const mi_tensor * b,
                          const mi_tensor * gate, const mi_tensor * norm_w, const mi_tensor * scale,
                          const mi_tensor * shift, float eps, const mi_tensor * sum, const mi_tensor * y,
                          void * workspace, size_t workspace_bytes, mi_stream stream);

/* The DiT sampler's per-step math on the device (dit_ggml_generate,
 * dit-sampler.h:408-640), so the latents stay resident across steps.
 * Latents and velocities are F32 [Oc, T, N], contiguous.
 * mi_apg_forward: apg_forward (dit-sampler.h:66-118) for N samples at once,
 *   in double: momentum running average (APGMomentumBuffer, 19-35; momentum
 *   -0.75 in the reference), per-channel L2 clip over T to norm_threshold
 *   (2.5), projection onto pred_cond (apg_project, 37-64), out = cond +
 *   (scale - 1) * orthogonal. momentum_buf: device memory of
 *   mi_apg_buffer_bytes() (a double per element) kept across the steps of
 *   one generation; first = 1 on its first use (the buffer is then set).
 *   Oc <= 1024.
 * mi_flow_step: one solver step in place, x_next from x_t and v_t
 *   (solvers/solver-euler.h: xt -= vt * (t_curr - t_next); solver-dpm.h:
 *   DPM++ 3M with `history` stored velocities in prev / prev2, Euler at 0 and
 *   AB2 at 1, then prev2 <- prev, prev <- vt; prev/prev2 ignored for Euler).
 * mi_flow_final: the last step, out = xt - vt * t (dit-sampler.h:601-605). */
enum { MI_SOLVER_EULER = 0, MI_SOLVER_DPM3M = 1 };
int mi_apg_buffer_bytes(const mi_tensor * cond, size_t * bytes);
int mi_apg_forward(const mi_tensor * cond, const mi_tensor * uncond, float guidance_scale, float momentum,
                   float norm_threshold, void * momentum_buf, size_t momentum_bytes, int first, const mi_tensor * out,
                   mi_stream stream);
int mi_flow_step(int solver, const mi_tensor * vt, const mi_tensor * xt, float t_curr, float t_next, int history,
                 const mi_tensor * prev, const mi_tensor * prev2, mi_stream stream);
int mi_flow_final(const mi_tensor * xt, const mi_tensor * vt, float t, const mi_tensor * out, mi_stream stream);

/* The other solvers of solvers/solver-registry.h:30-33 and the DCW correction.
 *
 * mi_flow_step_sde: the SDE ancestral step (solvers/solver-sde.h:17-38),
 *   x0 = xt - vt * t_curr; xt = t_next * noise + (1 - t_next) * x0, fp32 in
 *   that order. noise: F32 [Oc, T, N], the step's standard normal draws (the
 *   reference draws them on the host with Philox from seed_b + step + 1,
 *   philox.h; the caller brings them).
 *
 * mi_stork4_step: one STORK4 step (solvers/solver-stork.h:269-323) in place.
 *   history = velocities stored so far (0: the Euler bootstrap step, 289-296);
 *   prev / prev2 hold the latest two with their step sizes h_prev / h_prev2
 *   (the dt of the steps that stored them); on return prev2 <- prev and
 *   prev <- vt (the caller shifts h_prev2 <- h_prev, h_prev <- t_curr - t_next).
 *   Velocity derivatives by forward difference and the three-point formula
 *   with the reference's guards (69-126); ROCK4 sub-stepping of `substeps`
 *   (reference default 10; at least 2, clamped to the largest degree) halved
 *   while any result is not finite, then Euler (298-318). tables: the ROCK4
 *   coefficient tables, host memory (solver-stork4-constants.h:
 *   STORK4_MS / FPA / FPB / RECF), degrees ascending and <= 160.
 *   workspace: mi_stork4_workspace() bytes of device memory, 256-aligned, kept
 *   for the whole generation; its first four 32-bit words report the number
 *   of Euler fallbacks since the bootstrap step, the last step's derivative
 *   order, and the degree it accepted (0: Euler). Calls sharing a workspace race.
 *
 * mi_dcw: the Differential Correction in Wavelet domain after a solver step
 *   (dit-sampler.h:613-667, dwt-haar.h), per sample, in place:
 *   denoised = xt - vt * t_next; low: the Haar low band of xt moves by
 *   t_curr * scaler * (xL - yL); high: the high band by (1 - t_curr) * scaler;
 *   double: low by t_curr * scaler and high by (1 - t_curr) * high_scaler;
 *   pix: xt += scaler * (xt - denoised). A zero effective scaler leaves xt
 *   untouched. The reference applies it only to solvers that inject no noise. */
typedef struct mi_rock4_tables {
    const int32_t * ms;        /* [ms_len] degrees, ascending */
    const double *  fpa;       /* [ms_len][6] finishing coefficients A */
    const double *  fpb;       /* [ms_len][4] finishing coefficients B */
    const double *  recf;      /* [recf_len] recurrence coefficients */
    int32_t         ms_len;
    int32_t         recf_len;
} mi_rock4_tables;
enum { MI_DCW_LOW = 0, MI_DCW_HIGH = 1, MI_DCW_DOUBLE = 2, MI_DCW_PIX = 3 };
int mi_flow_step_sde(const mi_tensor * vt, const mi_tensor * xt, const mi_tensor * noise, float t_curr, float t_next,
                     mi_stream stream);
int mi_stork4_workspace(const mi_tensor * xt, size_t * bytes);
int mi_stork4_step(const mi_tensor * vt, const mi_tensor * xt, float t_curr, float t_next, int history, float h_prev,
                   float h_prev2, const mi_tensor * prev, const mi_tensor * prev2, int substeps,
                   const mi_rock4_tables * tables, void * workspace, size_t workspace_bytes, mi_stream stream);
int mi_dcw(int mode, const mi_tensor * xt, const mi_tensor * vt, float t_curr, float t_next, float scaler,
           float high_scaler, mi_stream stream);

/* GGUF reader and load-time weight preparation. Replaces gf_load (mmap, the
 * header parse and the check that every tensor lies inside the file,
 * gguf-weights.h:74-154), gf_load_tensor / gf_load_tensor_f32 (156-268),
 * gf_load_qkv_fused / gf_load_pair_fused (270-352) and gf_get_u32 / f32 /
 * str / bool (354-390). GGUF versions 2 and 3; tensor types with a known ggml
 * block size (F32, F16, BF16, Q4_0..Q8_1, Q2_K..Q8_K, I8..I64, F64; other
 * types: MI_ERR_TYPE). Malformed, truncated or misaligned files, and duplicate
 * keys or tensor names, return MI_ERR_FILE. The handle keeps the file mapped;
 * names, strings and tensor data pointers stay valid until mi_gguf_close. */
typedef struct mi_gguf mi_gguf;
typedef struct {
    const char * name;
    int32_t      type;    /* enum ggml_type */
    int32_t      n_dims;  /* 1..4 */
    int64_t      ne[4];   /* ggml order, 1 past n_dims */
    uint64_t     nbytes;
    const void * data;    /* host pointer into the mapped file */
} mi_gguf_tensor;

int     mi_gguf_open(const char * path, mi_gguf ** out);
void    mi_gguf_close(mi_gguf * g);
int64_t mi_gguf_n_tensors(const mi_gguf * g);
int64_t mi_gguf_find_tensor(const mi_gguf * g, const char * name); /* -1 if absent */
int     mi_gguf_get_tensor(const mi_gguf * g, int64_t idx, mi_gguf_tensor * t);
int64_t mi_gguf_n_kv(const mi_gguf * g);
int64_t mi_gguf_find_key(const mi_gguf * g, const char * key); /* -1 if absent */
int     mi_gguf_get_key(const mi_gguf * g, int64_t idx, const char ** key, int32_t * gguf_type);
/* typed values: MI_ERR_PARAM if the key is absent (the reference's getters then
 * return 0 / 0.0 / "" / false), MI_ERR_TYPE if it holds another GGUF type */
int mi_gguf_get_u32(const mi_gguf * g, const char * key, uint32_t * v);
int mi_gguf_get_f32(const mi_gguf * g, const char * key, float * v);
int mi_gguf_get_bool(const mi_gguf * g, const char * key, int * v);
int mi_gguf_get_str(const mi_gguf * g, const char * key, const char ** v);
/* Copy a tensor's bytes to device memory; to_f32 widens an F16 or BF16 tensor
 * to F32 (F32 tensors copy as they are; other types: MI_ERR_TYPE). */
int mi_gguf_upload(const mi_gguf * g, const char * name, int to_f32, void * dst, size_t dst_bytes, mi_stream stream);
/* Concatenate the rows of n 1-D/2-D tensors that share ne0 and type into dst
 * (q rows || k rows || v rows, or gate || up); *ne1_out = the summed ne1.
 * Different types: MI_ERR_UNSUPPORTED (load them separately, as the reference
 * falls back to). Calls return after the copies complete. */
int mi_gguf_upload_rows(const mi_gguf * g, const char * const * names, int n, void * dst, size_t dst_bytes,
                        int64_t * ne1_out, mi_stream stream);

/* ---------------------------------------------------------------------- */
/* Layer-chain drivers: launch the fused-op sequence of one DiT block or   */
/* one Qwen3 layer in the order of the reference's layer composers, taking */
/* the GEMM / attention outputs (not computed by this library) as inputs.  */
/* Every operand of the whole chain is validated before the first launch:  */
/* a non-zero return means nothing was launched and no buffer was written. */

/* One ACE-Step DiT block's non-GEMM ops, in dit_ggml_build_layer order
 * (dit-graph.h:367-448). hidden is updated in place. Each residual add is
 * fused with the RMSNorm that reads it (mi_add_rms_norm), so the block runs
 * as 5 launches without cross attention (8 with, both CA norms given):
 *   pre-SA:   norm_sa   = rms_norm_modulate(hidden, sa_norm_w, scale_sa, shift_sa)
 *   SA:       q_out/k_out = qk_norm_rope(q, k)   [q, k: views of the QKV GEMM output]
 *   post-SA:  hidden    = hidden + sa_out * gate_sa, fused with
 *               norm_ca  = rms_norm(hidden) * ca_norm_w            (cross attention), or
 *               norm_ffn = rms_norm_modulate(hidden, ffn_norm_w, scale_ffn, shift_ffn)
 *   CA:       ca_q_out  = rms_norm(ca_q) * ca_q_w   (when ca_q.data != NULL)
 *             ca_k_out  = rms_norm(ca_k) * ca_k_w   (when ca_k.data != NULL)
 *             hidden    = hidden + ca_out, fused with norm_ffn as above
 *   FFN:      ff        = swiglu(gate_up)
 *   post-FFN: hidden    = hidden + ffn_out * gate_ffn
 * adaln: F32 [6H] = scale_shift_table + tproj (shift_sa, scale_sa, gate_sa,
 * shift_ffn, scale_ffn, gate_ffn), as built at dit-graph.h:383-400. */
typedef struct mi_dit_block_io {
    mi_tensor hidden;                    /* [H, S, N] in/out */
    mi_tensor adaln;                     /* F32 [6H] */
    mi_tensor sa_norm_w, ffn_norm_w;     /* F32 [H] */
    mi_tensor norm_sa;                   /* [H, S, N] out */
    mi_tensor q, k, q_w, k_w, q_out, k_out, pos; /* self-attn QK-norm + rope */
    mi_tensor sa_out;                    /* [H, S, N] O-projection output */
    mi_tensor ca_norm_w, norm_ca;        /* cross-attn norm (optional) */
    mi_tensor ca_q, ca_q_w, ca_q_out;    /* cross-attn Q-norm (optional), dit-graph.h:328-329 */
    mi_tensor ca_out;                    /* cross-attn output (optional) */
    mi_tensor ca_k, ca_k_w, ca_k_out;    /* cross-attn K-norm (optional), dit-graph.h:330-331 */
    mi_tensor norm_ffn;                  /* [H, S, N] out */
    mi_tensor gate_up, ff;               /* [2I, S, N] -> [I, S, N] */
    mi_tensor ffn_out;                   /* [H, S, N] down-projection output */
    float     eps, rope_freq_base;
    int       n_dims;
    int       use_cross_attn;
} mi_dit_block_io;

int mi_dit_block_ops(const mi_dit_block_io * io, mi_stream stream);

/* One Qwen3 decoder layer's non-GEMM ops in qw3lm_forward_batch order
 * (qwen3-lm.h:630-741):
 *   norm   = rms_norm(hidden) * in_norm_w
 *   q/k    = qk_norm_rope(q, k)                [views of the QKV GEMM output]
 *   (clamp v in place when clamp_fp16), kv_store(k_out, v -> caches at pos0/sets)
 *     (with a cache and k_out.data NULL these are one mi_qk_norm_rope_kv_store
 *     launch instead: K goes only to the cache, and v is left unclamped in
 *     place; the cache gets the clamped values either way. That launch has
 *     mi_qk_norm_rope_kv_store's limits: for partial rotation (n_dims < D),
 *     D outside {64, 128, 256} or q/k/v views that are not 16-byte aligned,
 *     pass a k_out buffer, which selects the three-call path; without one
 *     such a layer returns MI_ERR_UNSUPPORTED before any launch)
 *   hidden = hidden + attn_out   (clamped to +-65504 when clamp_fp16), fused with
 *   norm2  = rms_norm(hidden) * post_norm_w
 *   ff     = swiglu(gate_up)
 *   hidden = hidden + mlp_out    (clamped when clamp_fp16) */
typedef struct mi_qwen3_layer_io {
    mi_tensor hidden;                       /* [H, n_tok] in/out */
    mi_tensor in_norm_w, post_norm_w;       /* F32 [H] */
    mi_tensor norm, norm2;                  /* [H, n_tok] out */
    mi_tensor q, k, v, q_w, k_w, q_out, k_out, pos;
    mi_tensor k_cache, v_cache, pos0, sets; /* optional KV store (k_cache.data NULL = skip) */
    mi_tensor attn_out;                     /* [H, n_tok] O-projection output */
    mi_tensor gate_up, ff;                  /* [2I, n_tok] -> [I, n_tok] */
    mi_tensor mlp_out;                      /* [H, n_tok] */
    float     eps, rope_freq_base;
    int       n_dims;
    int       clamp_fp16;
    int       kv_rounding;
    int32_t * d_err;
} mi_qwen3_layer_io;

int mi_qwen3_layer_ops(const mi_qwen3_layer_io * io, mi_stream stream);

#ifdef __cplusplus
}
#endif

#endif /* MI_OPS_H */
