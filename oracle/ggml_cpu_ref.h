/*
 * ggml_cpu_ref.h -- CPU oracle for the per-layer fused ops.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the ggml-cpu
 * arithmetic that acestep.cpp's graph builders invoke (ggml itself is an
 * empty submodule in the reference checkout, so it cannot be built here).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the parity reference or the timed CPU baseline --
 * never as part of the product path.
 *
 * Every function is one ggml graph node, computed the way ggml-cpu computes
 * it; composite chains are built by calling these in the order the
 * reference's graph builders emit them (see oracle/oracle.py).
 *
 * Layout convention: row-major, contiguous; "rows x n" means n is the
 * innermost (ggml ne0) dimension.
 *
 * Pinning (tests/test_oracle_pinning.py; each check is independent of the
 * formula restated here and fails on a planted mistake): fp16/bf16
 * conversions against numpy float16 and a nearest-neighbour search;
 * rms_norm against float64, exact rational arithmetic on tiny rows and
 * bit-exact power-of-two scaling; add/mul/clamp against single IEEE ops and
 * the NaN -> hi clamp semantics; rope by position-0 identity, pair norms,
 * the fp32 theta chain (and its divergence from the closed form at p = 8191),
 * partial n_dims, attn/freq scale; swiglu against float64 and IEEE special
 * values; Q8_0 by brute-force dequant, quantizer invariants and tie blocks
 * that separate the two variants; timestep embedding against float64 with a
 * derived bound; flash attention by one-key, equal-score and scale-0 closed
 * forms, key-permutation and GQA-mapping invariants, mask exclusion and the
 * q-conversion idempotence. Parity unpinned (needs the absent ggml source):
 * which Q8_0 variant ggml-cpu's ggml_cpy uses on x86 (both are implemented;
 * X86 is the default), the lane results of ggml's SIMD expf in swiglu,
 * whether the fork's CPU backend fuses nodes, and its FP-contraction flags;
 * for flash attention, ggml-cpu's own rounding (its SIMD dot products, and
 * the fp16 accumulation of the output when V is F16): orc_flash_attn_ext
 * states the exact value those roundings approximate.
 */
#ifndef ORC_GGML_CPU_REF_H
#define ORC_GGML_CPU_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- threading (rows are independent; results do not depend on it) ---- */
void orc_set_threads(int n);
int  orc_get_threads(void);

/* ---- number formats ---- */
float    orc_fp16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_fp16(float f);
float    orc_bf16_to_fp32(uint16_t h);
uint16_t orc_fp32_to_bf16(float f);
void     orc_fp16_to_fp32_n(const uint16_t * x, float * y, int64_t n);
void     orc_fp32_to_fp16_n(const float * x, uint16_t * y, int64_t n);
void     orc_bf16_to_fp32_n(const uint16_t * x, float * y, int64_t n);
void     orc_fp32_to_bf16_n(const float * x, uint16_t * y, int64_t n);

/* ---- ggml_rms_norm: y = x * (1/sqrtf(mean(x^2) + eps)), per row of n ---- */
void orc_rms_norm_f32(const float * x, int64_t rows, int64_t n, float eps, float * y);

/* ---- ggml binary ops with ggml_can_repeat broadcasting of b.
 *      a: rows x n; b: brows x bn with rows % brows == 0, n % bn == 0;
 *      b index = (r % brows, i % bn).  (ggml_add / ggml_mul) ---- */
void orc_add_f32(const float * a, const float * b, int64_t rows, int64_t n, int64_t brows, int64_t bn, float * y);
void orc_mul_f32(const float * a, const float * b, int64_t rows, int64_t n, int64_t brows, int64_t bn, float * y);

/* ---- ggml_clamp: y = MAX(MIN(x, hi), lo) ---- */
void orc_clamp_f32(const float * x, int64_t n, float lo, float hi, float * y);

/* ---- ggml_scale: y = x * s ---- */
void orc_scale_f32(const float * x, int64_t n, float s, float * y);

/* ---- ggml_rope_ext, mode NEOX (2), no freq_factors.
 *      x: n_pos x heads x ne0 (ggml [ne0, heads, n_pos]); rotates the first
 *      n_dims of each head row, copies the rest.  pos[n_pos] int32.
 *      ext_factor must be 0 (the only value the reference passes). ---- */
void orc_rope_neox_f32(const float * x, int64_t n_pos, int64_t heads, int64_t ne0, int n_dims, const int32_t * pos,
                       float freq_base, float freq_scale, float attn_factor, float * y);

/* theta_scale exactly as ggml-cpu derives it: powf(freq_base, -2.0f/n_dims) */
float orc_rope_theta_scale(float freq_base, int n_dims);

/* ---- ggml_swiglu / ggml_swiglu_split: y = silu(g) * u, silu(x) = x/(1+expf(-x)).
 *      g, u: rows x n with row strides gs, us (elements). ---- */
void orc_swiglu_f32(const float * g, int64_t gs, const float * u, int64_t us, int64_t rows, int64_t n, float * y);

/* ---- Q8_0 (block of 32: fp16 d, int8 qs[32]; 34 bytes) ---- */
#define ORC_QK8_0     32
#define ORC_Q8_0_SIZE 34
/* quantize_row_q8_0_ref: d = amax/127, id = d ? 1/d : 0, q = roundf(x*id) */
void orc_quantize_row_q8_0_ref(const float * x, uint8_t * y, int64_t k);
/* x86 from_float (AVX2 path): d = amax/127, id = amax ? 127/amax : 0, q = rint(x*id) */
void orc_quantize_row_q8_0_x86(const float * x, uint8_t * y, int64_t k);
void orc_dequantize_row_q8_0(const uint8_t * x, float * y, int64_t k);
/* rows x n floats -> rows x (n/32*34) bytes; variant 0 = ref, 1 = x86 */
void orc_quantize_rows_q8_0(const float * x, int64_t rows, int64_t n, int variant, uint8_t * y);

/* ---- ggml_get_rows: table n_rows x n (row bytes = row_size), ids[n_ids]
 *      -> y n_ids x n floats.  type: 0 = F32, 1 = F16, 8 = Q8_0, 30 = BF16.
 *      Returns -1 (and writes nothing for that row) on an out-of-range id. ---- */
int orc_get_rows(const void * table, int type, int64_t n_rows, int64_t n, const int32_t * ids, int64_t n_ids,
                 float * y);

/* ---- ggml_timestep_embedding: t[n] -> y n x dim ---- */
void orc_timestep_embedding_f32(const float * t, int64_t n, int dim, int max_period, float * y);

/* ---- ggml_flash_attn_ext(q, k, v, mask, scale, max_bias = 0, logit_softcap = 0)
 *      (dit-graph.h:227-231, 348-349; qwen3-lm.h:718-723), the exact
 *      mathematics of ggml-cpu's definition, in double:
 *        qc = q converted to K's vec_dot type: qconv 0 none (F32 K), 1 fp16
 *             (F16 K), 2 bf16 (BF16 K), 3 Q8_0 x86 quantize+dequantize (Q8_0 K)
 *        s_j = scale * dot(qc, k_j) + mask_j ; keys with mask_j == -inf skipped
 *        y   = sum_j exp(s_j - max) v_j / sum_j exp(s_j - max)
 *      A row whose keys are all masked gives NaN (ggml: 0 * (1/0)).
 *      q: [N][Nh][n_q][D], k, v: [N][Nkv][n_kv][D] (already dequantized to
 *      F32), mask: [mN][mH][mQ][n_kv] (F32 values of the F16 mask; index
 *      (b % mN, h % mH, iq)) or NULL, y: [N][n_q][Nh][D] (ggml's permuted
 *      result [D, Nh, n_q, N]). Head h reads KV head h / (Nh / Nkv). D <= 1024. ---- */
void orc_flash_attn_ext(const float * q, const float * k, const float * v, const float * mask, int64_t N, int64_t Nh,
                        int64_t Nkv, int64_t n_q, int64_t n_kv, int64_t D, int64_t mN, int64_t mH, int64_t mQ,
                        float scale, int qconv, float * y);
void orc_flash_attn_ext_f16acc(const float * q, const float * k, const uint16_t * v16, const float * mask,
                               int64_t N, int64_t Nh, int64_t Nkv, int64_t n_q, int64_t n_kv, int64_t D, int64_t mN,
                               int64_t mH, int64_t mQ, float scale, int qconv, float * y, float * bud);

/* ---- ggml_mul_mat(w, x), Q8_0 weights (qwen3-enc.h:86-88; dit-graph.h:36-49;
 *      qwen3-lm.h:755): w n rows of k / 32 Q8_0 blocks, x m rows of k F32,
 *      y m rows of n. Each row of x is quantized with the x86 quantizer (the
 *      vec_dot type's from_float); y is the exact value, in double, of
 *      sum_b fp16(d_w) fp16(d_x) sum_i q_w q_x, rounded to float once. ---- */
void orc_mul_mat_q8_0(const uint8_t * w, const float * x, int64_t n, int64_t k, int64_t m, float * y);

/* ---- DiT sampler step math (dit-sampler.h:19-118, 601-605; solvers/): APG in
 *      double with channel sums over T in order; Euler / DPM++ 3M steps
 *      (solver 0 / 1, hist = stored velocities) and the final x0 step in fp32,
 *      without contraction. Layout [n][t][oc]; ra is the momentum buffer. ---- */
void orc_apg_forward(const float * cond, const float * uncond, int64_t n, int64_t t, int64_t oc, float scale,
                     double momentum, float threshold, double * ra, int first, float * out);
void orc_flow_step(int solver, float * xt, const float * vt, int64_t n, float t_curr, float t_next, int hist,
                   float * prev, float * prev2);
void orc_flow_final(const float * xt, const float * vt, int64_t n, float t, float * out);

/* ---- The other sampler steps: SDE ancestral (solvers/solver-sde.h:17-38)
 *      with the step's N(0,1) draws given as noise; STORK4
 *      (solvers/solver-stork.h:269-323) over ROCK4 tables (degrees ms,
 *      finishing coefficients fpa [ms_len][6] / fpb [ms_len][4], recurrence
 *      coefficients recf), prev/prev2 = the two latest velocities with step
 *      sizes h1/h2, rotated on return; info[3] = derivative order, accepted
 *      degree (0 = Euler), Euler fallback flag. DCW (dit-sampler.h:613-667,
 *      dwt-haar.h) on [n][t][oc], mode 0 low, 1 high, 2 double, 3 pix. ---- */
typedef struct orc_rock4 {
    const int32_t * ms;
    const double *  fpa;
    const double *  fpb;
    const double *  recf;
    int             ms_len, recf_len;
} orc_rock4;
void orc_sde_step(float * xt, const float * vt, const float * noise, int64_t n, float t_curr, float t_next);
void orc_stork4_step(float * xt, const float * vt, int64_t n, float t_curr, float t_next, int hist, float h1,
                     float h2, float * prev, float * prev2, int substeps, const orc_rock4 * tab, int * info);
void orc_dcw(int mode, float * xt, const float * vt, int64_t n, int64_t t, int64_t oc, float t_curr, float t_next,
             float scaler, float high_scaler);

#ifdef __cplusplus
}
#endif

#endif
