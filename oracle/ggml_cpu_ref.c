/*
 * ggml_cpu_ref.c -- CPU oracle for the per-layer fused ops.
 *
 * TEST INFRASTRUCTURE ONLY (see ggml_cpu_ref.h). Not shipped, never on the
 * product path.
 *
 * This restates, node by node, the ggml-cpu arithmetic behind the ops that
 * acestep.cpp's graph builders emit. ggml is an empty submodule in the
 * reference checkout (.gitmodules:1-3), so each function below follows the
 * published ggml-cpu algorithm for that node; the reference call sites it
 * serves are cited per function. Build with -ffp-contract=off and without
 * -ffast-math so that every multiply/add rounds exactly as written.
 */
#include "ggml_cpu_ref.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 1;

void orc_set_threads(int n) {
    g_threads = n < 1 ? 1 : n;
}

int orc_get_threads(void) {
    return g_threads;
}

/* ------------------------------------------------------------------------ */
/* number formats                                                           */
/* ------------------------------------------------------------------------ */

static inline uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* IEEE binary16 -> binary32, exact (subnormals included). */
float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t e    = (h >> 10) & 0x1fu;
    const uint32_t m    = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: value = m * 2^-24 (exact in binary32) */
        const float v = (float) m * 0x1p-24f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) {
        return u2f(sign | 0x7f800000u | (m << 13));
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* binary32 -> binary16, round to nearest even, overflow to inf, NaN kept quiet. */
uint16_t orc_fp32_to_fp16(float f) {
    const uint32_t x    = f2u(f);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax   = x & 0x7fffffffu;
    if (ax > 0x7f800000u) {
        return (uint16_t) (sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) { /* >= 65520: the halfway point to 2^16 rounds (to even) up to inf */
        return (uint16_t) (sign | 0x7c00u);
    }
    if (ax >= 0x38800000u) { /* normal binary16 range, >= 2^-14 */
        const uint32_t e   = (ax >> 23) - 112u;
        const uint32_t m   = ax & 0x7fffffu;
        uint32_t       h   = (e << 10) | (m >> 13);
        const uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) {
            h++; /* a carry into the exponent is the correct result */
        }
        return (uint16_t) (sign | h);
    }
    if (ax <= 0x33000000u) { /* <= 2^-25: rounds to zero (2^-25 itself is a tie to even 0) */
        return sign;
    }
    /* subnormal binary16: k = round(|f| * 2^24), k in [1, 1024] */
    const uint32_t m   = (ax & 0x7fffffu) | 0x800000u;
    const int      E   = (int) (ax >> 23) - 127;      /* -25 .. -15 */
    const int      s   = -E - 1;                       /* 14 .. 24 */
    uint32_t       k   = m >> s;
    const uint32_t rem = m & ((1u << s) - 1u);
    const uint32_t half = 1u << (s - 1);
    if (rem > half || (rem == half && (k & 1u))) {
        k++;
    }
    return (uint16_t) (sign | k);
}

float orc_bf16_to_fp32(uint16_t h) {
    return u2f((uint32_t) h << 16);
}

/* binary32 -> bfloat16, round to nearest even; NaN is quieted. */
uint16_t orc_fp32_to_bf16(float f) {
    const uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t) ((u >> 16) | 64u);
    }
    return (uint16_t) ((u + (0x7fffu + ((u >> 16) & 1u))) >> 16);
}

void orc_fp16_to_fp32_n(const uint16_t * x, float * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = orc_fp16_to_fp32(x[i]);
    }
}

void orc_fp32_to_fp16_n(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = orc_fp32_to_fp16(x[i]);
    }
}

void orc_bf16_to_fp32_n(const uint16_t * x, float * y, int64_t n) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        y[i] = orc_bf16_to_fp32(x[i]);
    }
}

void orc_fp32_to_bf16_n(const float * x, uint16_t * y, int64_t n) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        y[i] = orc_fp32_to_bf16(x[i]);
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_rms_norm                                                            */
/* Reference call sites: qwen3-enc.h:118 (qwen3_rms_norm), 165-168 (QK-norm),*/
/* qwen3-lm.h:372-375, 660-663; dit-graph.h:28 (dit_ggml_rms_norm_weighted), */
/* 183-186, 328-331.                                                         */
/* Arithmetic (ggml-cpu rms_norm_f32): float square, double sequential sum,  */
/* mean = (float)(sum/n), scale = 1.0f/sqrtf(mean + eps), y = x * scale.     */
/* ------------------------------------------------------------------------ */
void orc_rms_norm_f32(const float * x, int64_t rows, int64_t n, float eps, float * y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float * xr  = x + r * n;
        float *       yr  = y + r * n;
        double        sum = 0.0;
        for (int64_t i = 0; i < n; i++) {
            sum += (double) (xr[i] * xr[i]);
        }
        const float mean  = (float) (sum / (double) n);
        const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < n; i++) {
            yr[i] = xr[i] * scale;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_add / ggml_mul with broadcast of b (ggml_can_repeat(b, a)).          */
/* Call sites: qwen3-enc.h:119 (norm * w), 238, 243 (residual add);          */
/* qwen3-lm.h:479, 487, 730, 738; dit-graph.h:29, 61-63 (AdaLN), 74-75       */
/* (gated residual), 391 (AdaLN vectors), 432.                              */
/* ------------------------------------------------------------------------ */
void orc_add_f32(const float * a, const float * b, int64_t rows, int64_t n, int64_t brows, int64_t bn, float * y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float * br = b + (r % brows) * bn;
        for (int64_t i = 0; i < n; i++) {
            y[r * n + i] = a[r * n + i] + br[i % bn];
        }
    }
}

void orc_mul_f32(const float * a, const float * b, int64_t rows, int64_t n, int64_t brows, int64_t bn, float * y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float * br = b + (r % brows) * bn;
        for (int64_t i = 0; i < n; i++) {
            y[r * n + i] = a[r * n + i] * br[i % bn];
        }
    }
}

/* ggml_clamp (qwen3-lm.h:393, 481, 489, 676, 732, 740): MAX(MIN(x, hi), lo)
 * with the C-macro comparisons, so a NaN input yields hi. */
void orc_clamp_f32(const float * x, int64_t n, float lo, float hi, float * y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float a = x[i] < hi ? x[i] : hi;
        y[i]          = a > lo ? a : lo;
    }
}

/* ggml_scale (dit-graph.h:87): y = x * s */
void orc_scale_f32(const float * x, int64_t n, float s, float * y) {
    for (int64_t i = 0; i < n; i++) {
        y[i] = x[i] * s;
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_rope_ext, mode 2 (NEOX).                                             */
/* Call sites: qwen3-enc.h:173-174, qwen3-lm.h:378-379, 666-667,             */
/* dit-graph.h:194-196 (all: n_dims = D, n_ctx_orig = 0, freq_scale = 1,     */
/* ext_factor = 0, attn_factor = 1, beta_fast = beta_slow = 0).              */
/* Arithmetic (ggml-cpu rope): theta_scale = powf(base, -2/n_dims); per      */
/* position the angle starts at (float)p and is multiplied by theta_scale    */
/* once per pair (an iterative fp32 chain); cos/sin are libm cosf/sinf       */
/* scaled by attn_factor; pair (i, i + n_dims/2) is rotated.                 */
/* ------------------------------------------------------------------------ */
float orc_rope_theta_scale(float freq_base, int n_dims) {
    return powf(freq_base, -2.0f / (float) n_dims);
}

void orc_rope_neox_f32(const float * x, int64_t n_pos, int64_t heads, int64_t ne0, int n_dims, const int32_t * pos,
                       float freq_base, float freq_scale, float attn_factor, float * y) {
    const float   theta_scale = orc_rope_theta_scale(freq_base, n_dims);
    const int64_t half        = n_dims / 2;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t t = 0; t < n_pos; t++) {
        float cache[2 * 4096];
        float theta = (float) pos[t];
        for (int64_t i0 = 0; i0 < ne0 && i0 < 2 * 4096; i0 += 2) {
            const float th = freq_scale * theta; /* rope_yarn with ext_factor == 0 */
            cache[i0 + 0]  = cosf(th) * attn_factor;
            cache[i0 + 1]  = sinf(th) * attn_factor;
            theta *= theta_scale;
        }
        for (int64_t h = 0; h < heads; h++) {
            const float * src = x + (t * heads + h) * ne0;
            float *       dst = y + (t * heads + h) * ne0;
            for (int64_t ic = 0; ic < half; ic++) {
                const float c  = cache[2 * ic + 0];
                const float s  = cache[2 * ic + 1];
                const float x0 = src[ic];
                const float x1 = src[ic + half];
                dst[ic]        = x0 * c - x1 * s;
                dst[ic + half] = x0 * s + x1 * c;
            }
            for (int64_t i0 = n_dims; i0 < ne0; i0++) {
                dst[i0] = src[i0];
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_swiglu (fused [2I] input, gate = first half) and ggml_swiglu_split.  */
/* Call sites: qwen3-enc.h:217, 221; dit-graph.h:259, 264.                   */
/* Arithmetic: ggml_silu_f32(g) * u with silu(x) = x/(1.0f + expf(-x)) (the  */
/* scalar form; ggml's SIMD lanes use a polynomial expf whose lane results   */
/* cannot be reproduced without the ggml source: within ~1e-7 relative).     */
/* ------------------------------------------------------------------------ */
void orc_swiglu_f32(const float * g, int64_t gs, const float * u, int64_t us, int64_t rows, int64_t n, float * y) {
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float * gr = g + r * gs;
        const float * ur = u + r * us;
        float *       yr = y + r * n;
        for (int64_t i = 0; i < n; i++) {
            const float xg = gr[i];
            yr[i]          = (xg / (1.0f + expf(-xg))) * ur[i];
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_0. Block = { fp16 d; int8 qs[32] }, 34 bytes, no padding.              */
/* Writers: the Q8_0 KV cache ggml_cpy at songgen-lelm-gen.h:254-265 and     */
/* 548-562 (SG_KV_TYPE=q8_0, 53-61); the Q8_0 embedding tables written by    */
/* tools/quantize.cpp (ggml_quantize_chunk -> quantize_row_q8_0_ref).        */
/* ------------------------------------------------------------------------ */
static inline float round_half_away(float v) {
    return roundf(v);
}

static inline float round_half_even(float v) {
    return rintf(v); /* default FE_TONEAREST */
}

void orc_quantize_row_q8_0_ref(const float * x, uint8_t * y, int64_t k) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb   = x + i * ORC_QK8_0;
        uint8_t *     yb   = y + i * ORC_Q8_0_SIZE;
        float         amax = 0.0f;
        for (int j = 0; j < ORC_QK8_0; j++) {
            const float v = fabsf(xb[j]);
            amax          = amax > v ? amax : v;
        }
        const float    d   = amax / 127.0f;
        const float    id  = d != 0.0f ? 1.0f / d : 0.0f;
        const uint16_t d16 = orc_fp32_to_fp16(d);
        memcpy(yb, &d16, 2);
        for (int j = 0; j < ORC_QK8_0; j++) {
            yb[2 + j] = (uint8_t) (int8_t) round_half_away(xb[j] * id);
        }
    }
}

void orc_quantize_row_q8_0_x86(const float * x, uint8_t * y, int64_t k) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float * xb   = x + i * ORC_QK8_0;
        uint8_t *     yb   = y + i * ORC_Q8_0_SIZE;
        float         amax = 0.0f;
        for (int j = 0; j < ORC_QK8_0; j++) {
            const float v = fabsf(xb[j]);
            amax          = amax > v ? amax : v;
        }
        const float    d   = amax / 127.0f;
        const uint16_t d16 = orc_fp32_to_fp16(d);
        const float    id  = amax != 0.0f ? 127.0f / amax : 0.0f;
        memcpy(yb, &d16, 2);
        for (int j = 0; j < ORC_QK8_0; j++) {
            float q = round_half_even(xb[j] * id);
            /* packs_epi32 / packs_epi16 saturate */
            q         = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
            yb[2 + j] = (uint8_t) (int8_t) q;
        }
    }
}

void orc_dequantize_row_q8_0(const uint8_t * x, float * y, int64_t k) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const uint8_t * xb = x + i * ORC_Q8_0_SIZE;
        uint16_t        d16;
        memcpy(&d16, xb, 2);
        const float d = orc_fp16_to_fp32(d16);
        for (int j = 0; j < ORC_QK8_0; j++) {
            y[i * ORC_QK8_0 + j] = (float) (int8_t) xb[2 + j] * d;
        }
    }
}

void orc_quantize_rows_q8_0(const float * x, int64_t rows, int64_t n, int variant, uint8_t * y) {
    const int64_t rb = n / ORC_QK8_0 * ORC_Q8_0_SIZE;
#pragma omp parallel for num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        if (variant == 0) {
            orc_quantize_row_q8_0_ref(x + r * n, y + r * rb, n);
        } else {
            orc_quantize_row_q8_0_x86(x + r * n, y + r * rb, n);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_get_rows (qwen3-enc.h:390, 465; qwen3-lm.h:464, 626): one table row  */
/* per id, dequantized/converted to F32 (ggml-cpu get_rows_q / _f16 / _bf16).*/
/* ------------------------------------------------------------------------ */
int orc_get_rows(const void * table, int type, int64_t n_rows, int64_t n, const int32_t * ids, int64_t n_ids,
                 float * y) {
    int64_t row_size;
    switch (type) {
        case 0:
            row_size = n * 4;
            break;
        case 1:
        case 30:
            row_size = n * 2;
            break;
        case 8:
            row_size = n / ORC_QK8_0 * ORC_Q8_0_SIZE;
            break;
        default:
            return -2;
    }
    int bad = 0;
#pragma omp parallel for num_threads(g_threads) schedule(static) reduction(| : bad)
    for (int64_t i = 0; i < n_ids; i++) {
        const int64_t r = ids[i];
        if (r < 0 || r >= n_rows) {
            bad = 1;
            continue;
        }
        const uint8_t * src = (const uint8_t *) table + r * row_size;
        float *         dst = y + i * n;
        switch (type) {
            case 0:
                memcpy(dst, src, (size_t) n * 4);
                break;
            case 1:
                orc_fp16_to_fp32_n((const uint16_t *) src, dst, n);
                break;
            case 30:
                for (int64_t j = 0; j < n; j++) {
                    dst[j] = orc_bf16_to_fp32(((const uint16_t *) src)[j]);
                }
                break;
            case 8:
                orc_dequantize_row_q8_0(src, dst, n);
                break;
        }
    }
    return bad ? -1 : 0;
}

/* ------------------------------------------------------------------------ */
/* ggml_timestep_embedding (dit-graph.h:90, dim 256, max_period 10000):      */
/* freq_j = expf(-logf(max_period) * j / half); out[j] = cosf(t*freq_j),     */
/* out[j + half] = sinf(t*freq_j); an odd dim leaves a trailing 0.           */
/* ------------------------------------------------------------------------ */
void orc_timestep_embedding_f32(const float * t, int64_t n, int dim, int max_period, float * y) {
    const int half = dim / 2;
    for (int64_t i = 0; i < n; i++) {
        float * e = y + i * dim;
        for (int64_t j = 0; j < half; j++) {
            const float timestep = t[i];
            const float freq     = expf(-logf((float) max_period) * (float) j / (float) half);
            const float arg      = timestep * freq;
            e[j]                 = cosf(arg);
            e[j + half]          = sinf(arg);
        }
        if (dim % 2 != 0) {
            e[2 * half] = 0.0f;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_flash_attn_ext (dit-graph.h:227-231, 348-349; qwen3-lm.h:718-723),  */
/* GGML_PREC_F32, max_bias = 0, logit_softcap = 0. ggml-cpu converts each q  */
/* row to K's vec_dot type before the dot products (fp16 for F16 K, bf16 for */
/* BF16 K, Q8_0 -- the arch from_float -- for Q8_0 K), skips keys whose mask */
/* is -inf, and runs an online softmax over the rest. This states the exact  */
/* value of that definition: products and sums in double, one softmax.      */
/* ------------------------------------------------------------------------ */
static void fa_convert_q(const float * q, int64_t D, int qconv, double * qc) {
    if (qconv == 3) {
        uint8_t blk[ORC_Q8_0_SIZE];
        float   deq[ORC_QK8_0];
        for (int64_t b = 0; b < D / ORC_QK8_0; b++) {
            orc_quantize_row_q8_0_x86(q + b * ORC_QK8_0, blk, ORC_QK8_0);
            orc_dequantize_row_q8_0(blk, deq, ORC_QK8_0);
            for (int j = 0; j < ORC_QK8_0; j++) {
                qc[b * ORC_QK8_0 + j] = deq[j];
            }
        }
        return;
    }
    for (int64_t d = 0; d < D; d++) {
        float x = q[d];
        if (qconv == 1) {
            x = orc_fp16_to_fp32(orc_fp32_to_fp16(x));
        } else if (qconv == 2) {
            x = orc_bf16_to_fp32(orc_fp32_to_bf16(x));
        }
        qc[d] = x;
    }
}

void orc_flash_attn_ext(const float * q, const float * k, const float * v, const float * mask, int64_t N, int64_t Nh,
                        int64_t Nkv, int64_t n_q, int64_t n_kv, int64_t D, int64_t mN, int64_t mH, int64_t mQ,
                        float scale, int qconv, float * y) {
    const int64_t rk = Nh / Nkv;
#pragma omp parallel for collapse(3) num_threads(g_threads) schedule(static)
    for (int64_t b = 0; b < N; b++) {
        for (int64_t h = 0; h < Nh; h++) {
            for (int64_t iq = 0; iq < n_q; iq++) {
                double        qc[1024];
                double        acc[1024];
                const int64_t g  = h / rk;
                const float * kk = k + (b * Nkv + g) * n_kv * D;
                const float * vv = v + (b * Nkv + g) * n_kv * D;
                const float * mm = mask ? mask + (((b % mN) * mH + (h % mH)) * mQ + iq) * n_kv : NULL;
                fa_convert_q(q + ((b * Nh + h) * n_q + iq) * D, D, qconv, qc);
                double smax = -INFINITY;
                for (int64_t j = 0; j < n_kv; j++) {
                    const double mv = mm ? (double) mm[j] : 0.0;
                    if (mv == -INFINITY) {
                        continue;
                    }
                    double dot = 0.0;
                    for (int64_t d = 0; d < D; d++) {
                        dot += qc[d] * (double) kk[j * D + d];
                    }
                    const double s = (double) scale * dot + mv;
                    smax           = s > smax ? s : smax;
                }
                double sum = 0.0;
                for (int64_t d = 0; d < D; d++) {
                    acc[d] = 0.0;
                }
                for (int64_t j = 0; j < n_kv; j++) {
                    const double mv = mm ? (double) mm[j] : 0.0;
                    if (mv == -INFINITY) {
                        continue;
                    }
                    double dot = 0.0;
                    for (int64_t d = 0; d < D; d++) {
                        dot += qc[d] * (double) kk[j * D + d];
                    }
                    const double p = exp((double) scale * dot + mv - smax);
                    sum += p;
                    for (int64_t d = 0; d < D; d++) {
                        acc[d] += p * (double) vv[j * D + d];
                    }
                }
                float * yo = y + ((b * n_q + iq) * Nh + h) * D;
                for (int64_t d = 0; d < D; d++) {
                    yo[d] = (float) (acc[d] * (1.0 / sum)); /* all masked: 0 * inf = NaN, as ggml */
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* The same op as ggml-cpu computes it for an F16 V (ggml upstream, not in    */
/* this checkout: ops.cpp ggml_compute_forward_flash_attn_ext_f16_one_chunk,  */
/* dbrain/ggml 292516d5): one key at a time, the score in float              */
/* (s = dot * scale + mask), M and S in float; the output accumulated in      */
/* FP16: on a new maximum VKQ16 *= ms = expf(Mold - M) (vs = 1), else          */
/* vs = expf(s - M); then VKQ16 += v * vs, each element rounded to fp16;     */
/* S = S * ms + vs; finally y = f32(VKQ16) * (1 / S). The dot is taken in     */
/* double and rounded to float (ggml's SIMD f32 lane order is not restated). */
/* bud receives, per output element, the fp16 rounding errors of VKQ16 as    */
/* they propagate to y (each rounding's exact size, carried through later    */
/* rescales, divided by S).                                                  */
/* ------------------------------------------------------------------------ */
void orc_flash_attn_ext_f16acc(const float * q, const float * k, const uint16_t * v16, const float * mask,
                               int64_t N, int64_t Nh, int64_t Nkv, int64_t n_q, int64_t n_kv, int64_t D, int64_t mN,
                               int64_t mH, int64_t mQ, float scale, int qconv, float * y, float * bud) {
    const int64_t rk = Nh / Nkv;
#pragma omp parallel for collapse(3) num_threads(g_threads) schedule(static)
    for (int64_t b = 0; b < N; b++) {
        for (int64_t h = 0; h < Nh; h++) {
            for (int64_t iq = 0; iq < n_q; iq++) {
                double          qc[1024];
                uint16_t        acc[1024];
                double          err[1024];
                const int64_t   g  = h / rk;
                const float *   kk = k + (b * Nkv + g) * n_kv * D;
                const uint16_t * vv = v16 + (b * Nkv + g) * n_kv * D;
                const float *   mm = mask ? mask + (((b % mN) * mH + (h % mH)) * mQ + iq) * n_kv : NULL;
                fa_convert_q(q + ((b * Nh + h) * n_q + iq) * D, D, qconv, qc);
                for (int64_t d = 0; d < D; d++) {
                    acc[d] = orc_fp32_to_fp16(0.0f);
                    err[d] = 0.0;
                }
                float S = 0.0f, M = -INFINITY;
                for (int64_t j = 0; j < n_kv; j++) {
                    const float mv = mm ? mm[j] : 0.0f;
                    if (mv == -INFINITY) {
                        continue;
                    }
                    double dot = 0.0;
                    for (int64_t d = 0; d < D; d++) {
                        dot += qc[d] * (double) kk[j * D + d];
                    }
                    float       sc   = (float) dot;
                    sc               = sc * scale;
                    sc               = sc + mv;
                    const float Mold = M;
                    float       ms = 1.0f, vs = 1.0f;
                    if (sc > M) {
                        M  = sc;
                        ms = expf(Mold - M);
                        for (int64_t d = 0; d < D; d++) {
                            const float x = orc_fp16_to_fp32(acc[d]) * ms;
                            acc[d]        = orc_fp32_to_fp16(x);
                            err[d]        = err[d] * ms + fabs((double) orc_fp16_to_fp32(acc[d]) - (double) x);
                        }
                    } else {
                        vs = expf(sc - M);
                    }
                    for (int64_t d = 0; d < D; d++) {
                        const float x = fmaf(orc_fp16_to_fp32(vv[j * D + d]), vs, orc_fp16_to_fp32(acc[d]));
                        acc[d]        = orc_fp32_to_fp16(x);
                        err[d] += fabs((double) orc_fp16_to_fp32(acc[d]) - (double) x);
                    }
                    S = S * ms + vs;
                }
                const float S_inv = 1.0f / S; /* all masked: 0 * inf = NaN, as the exact oracle */
                float *     yo    = y + ((b * n_q + iq) * Nh + h) * D;
                float *     bo    = bud + ((b * n_q + iq) * Nh + h) * D;
                for (int64_t d = 0; d < D; d++) {
                    yo[d] = orc_fp16_to_fp32(acc[d]) * S_inv;
                    bo[d] = (float) (err[d] / (double) S);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* ggml_mul_mat(w, x) with Q8_0 weights (qwen3-enc.h:86-88; dit-graph.h:36-49; */
/* qwen3-lm.h:755): ggml-cpu quantizes each row of x with the vec_dot type's  */
/* from_float (Q8_0, x86) and takes ggml_vec_dot_q8_0_q8_0 per output. Here   */
/* the exact value of that dot, in double: sum over blocks of                 */
/* fp16(d_w) * fp16(d_x) * (exact int32 sum of q_w * q_x).                    */
/* ------------------------------------------------------------------------ */
void orc_mul_mat_q8_0(const uint8_t * w, const float * x, int64_t n, int64_t k, int64_t m, float * y) {
    const int64_t nb = k / ORC_QK8_0;
    uint8_t *     xq = (uint8_t *) malloc((size_t) (m * nb * ORC_Q8_0_SIZE) + 1);
    for (int64_t r = 0; r < m; r++) {
        orc_quantize_row_q8_0_x86(x + r * k, xq + r * nb * ORC_Q8_0_SIZE, k);
    }
#pragma omp parallel for collapse(2) num_threads(g_threads) schedule(static)
    for (int64_t r = 0; r < m; r++) {
        for (int64_t j = 0; j < n; j++) {
            double s = 0.0;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t * wb = w + (j * nb + b) * ORC_Q8_0_SIZE;
                const uint8_t * xb = xq + (r * nb + b) * ORC_Q8_0_SIZE;
                uint16_t        dw, dx;
                memcpy(&dw, wb, 2);
                memcpy(&dx, xb, 2);
                int32_t isum = 0;
                for (int i = 0; i < ORC_QK8_0; i++) {
                    isum += (int32_t) (int8_t) wb[2 + i] * (int32_t) (int8_t) xb[2 + i];
                }
                s += (double) orc_fp16_to_fp32(dw) * (double) orc_fp16_to_fp32(dx) * (double) isum;
            }
            y[r * n + j] = (float) s;
        }
    }
    free(xq);
}

/* ------------------------------------------------------------------------ */
/* DiT sampler step math (dit-sampler.h): apg_forward (66-118) with its      */
/* momentum buffer (19-35) and apg_project (37-64), in double, channels      */
/* summed over T in order; Euler (solvers/solver-euler.h) and DPM++ 3M       */
/* (solvers/solver-dpm.h) steps and the final x0 step (601-605) in fp32.     */
/* Layout [n][t][oc].                                                        */
/* ------------------------------------------------------------------------ */
void orc_apg_forward(const float * cond, const float * uncond, int64_t n, int64_t t, int64_t oc, float scale,
                     double momentum, float threshold, double * ra, int first, float * out) {
    for (int64_t b = 0; b < n; b++) {
        const float * pc = cond + b * t * oc;
        const float * pu = uncond + b * t * oc;
        double *      r  = ra + b * t * oc;
        float *       y  = out + b * t * oc;
        const int64_t m  = t * oc;
        double *      d  = (double *) malloc((size_t) m * sizeof(double) + 8);
        for (int64_t i = 0; i < m; i++) {
            const double v = (double) pc[i] - (double) pu[i];
            r[i]           = first ? v : v + momentum * r[i];
            d[i]           = r[i];
        }
        if (threshold > 0.0f) {
            for (int64_t c = 0; c < oc; c++) {
                double n2 = 0.0;
                for (int64_t k = 0; k < t; k++) {
                    n2 += d[k * oc + c] * d[k * oc + c];
                }
                const double nrm = sqrt(n2 > 0.0 ? n2 : 0.0);
                const double sc  = nrm > 1e-60 ? fmin(1.0, (double) threshold / nrm) : 1.0;
                if (sc < 1.0) {
                    for (int64_t k = 0; k < t; k++) {
                        d[k * oc + c] *= sc;
                    }
                }
            }
        }
        const double w = (double) scale - 1.0;
        for (int64_t c = 0; c < oc; c++) {
            double n2 = 0.0;
            for (int64_t k = 0; k < t; k++) {
                n2 += (double) pc[k * oc + c] * (double) pc[k * oc + c];
            }
            const double inv = n2 > 1e-60 ? 1.0 / sqrt(n2) : 0.0;
            double       dot = 0.0;
            for (int64_t k = 0; k < t; k++) {
                dot += d[k * oc + c] * ((double) pc[k * oc + c] * inv);
            }
            for (int64_t k = 0; k < t; k++) {
                const int64_t i   = k * oc + c;
                const double  v1n = (double) pc[i] * inv;
                const double  orth = d[i] - dot * v1n;
                y[i]               = (float) ((double) pc[i] + w * orth);
            }
        }
        free(d);
    }
}

void orc_flow_step(int solver, float * xt, const float * vt, int64_t n, float t_curr, float t_next, int hist,
                   float * prev, float * prev2) {
    const float dt = t_curr - t_next;
    for (int64_t i = 0; i < n; i++) {
        float ve = vt[i];
        if (solver == 1) {
            if (hist >= 2) {
                const float c0 = 23.0f / 12.0f, c1 = 16.0f / 12.0f, c2 = 5.0f / 12.0f;
                ve = c0 * vt[i] - c1 * prev[i] + c2 * prev2[i];
            } else if (hist == 1) {
                ve = 1.5f * vt[i] - 0.5f * prev[i];
            }
        }
        const float p = ve * dt;
        xt[i]         = xt[i] - p;
    }
    if (solver == 1) {
        for (int64_t i = 0; i < n; i++) {
            if (hist >= 1) {
                prev2[i] = prev[i];
            }
            prev[i] = vt[i];
        }
    }
}

void orc_flow_final(const float * xt, const float * vt, int64_t n, float t, float * out) {
    for (int64_t i = 0; i < n; i++) {
        const float p = vt[i] * t;
        out[i]        = xt[i] - p;
    }
}

/* ------------------------------------------------------------------------ */
/* The other sampler steps: SDE ancestral (solvers/solver-sde.h:17-38) with  */
/* the step's standard normal draws given, STORK4 (solvers/solver-stork.h),  */
/* and DCW (dit-sampler.h:613-667 over dwt-haar.h). fp32 in the reference's  */
/* operation order, the derivative sums in double. Layout [n][t][oc].        */
/* ------------------------------------------------------------------------ */
void orc_sde_step(float * xt, const float * vt, const float * noise, int64_t n, float t_curr, float t_next) {
    /* solver-sde.h:33-36 */
    for (int64_t i = 0; i < n; i++) {
        const float x0 = xt[i] - vt[i] * t_curr;
        xt[i]          = t_next * noise[i] + (1.0f - t_next) * x0;
    }
}

/* _stork_rms (solver-stork.h:34-41): double sum in index order */
static double stork_rms(const float * d, int64_t n) {
    double s = 0.0;
    for (int64_t i = 0; i < n; i++) {
        s += (double) d[i] * (double) d[i];
    }
    return sqrt(s / (double) n);
}

/* _stork_taylor_approx (solver-stork.h:45-64) */
static void stork_taylor(float * out, int order, float diff, const float * v, const float * dv, const float * d2v,
                         int64_t n) {
    if (order >= 2) {
        const float h = 0.5f * diff * diff;
        for (int64_t i = 0; i < n; i++) {
            out[i] = v[i] + diff * dv[i] + h * d2v[i];
        }
    } else if (order == 1) {
        for (int64_t i = 0; i < n; i++) {
            out[i] = v[i] + diff * dv[i];
        }
    } else {
        memcpy(out, v, (size_t) n * sizeof(float));
    }
}

/* _stork_compute_derivatives (solver-stork.h:69-126) with the two most recent
 * records as (prev, h1) and (prev2, h2); hist = records stored (0, 1, 2+) */
static int stork_derivatives(const float * vt, int64_t n, int hist, const float * prev, float h1, const float * prev2,
                             float h2, float * dv, float * d2v) {
    if (hist < 1 || h1 == 0.0f) {
        return 0;
    }
    for (int64_t i = 0; i < n; i++) {
        dv[i] = (prev[i] - vt[i]) / h1;
    }
    const double vt_rms = stork_rms(vt, n);
    const double dv_rms = stork_rms(dv, n);
    if (vt_rms > 0.0 && dv_rms * fabs((double) h1) > 5.0 * vt_rms) {
        return 0;
    }
    if (hist < 2 || h2 == 0.0f) {
        return 1;
    }
    const double h1d = (double) h1, h2d = (double) h2;
    const double den = h1d * h2d * (h1d + h2d);
    if (fabs(den) < 1e-30) {
        return 1;
    }
    const double c = 2.0 / den;
    for (int64_t i = 0; i < n; i++) {
        d2v[i] = (float) (c * ((double) prev2[i] * h1d - (double) prev[i] * (h1d + h2d) + (double) vt[i] * h2d));
    }
    const double d2v_rms = stork_rms(d2v, n);
    if (vt_rms > 0.0 && d2v_rms * (double) h1 * (double) h1 > 5.0 * vt_rms) {
        return 1;
    }
    return 2;
}

/* _rock4_mdegr (solver-stork.h:140-159) */
static void rock4_mdegr(int s, const int32_t * ms, int ms_len, int * mdeg, int * mz, int * mr) {
    int mp1 = 1;
    for (int i = 0; i < ms_len; i++) {
        if (ms[i] >= s) {
            *mdeg = ms[i];
            *mz   = i;
            *mr   = mp1 - 1;
            return;
        }
        mp1 += ms[i] * 2 - 1;
    }
    *mz   = ms_len - 1;
    *mdeg = ms[*mz];
    *mr   = mp1 - 1;
}

static int all_finite(const float * x, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        if (!isfinite(x[i])) {
            return 0;
        }
    }
    return 1;
}

/* _rock4_substep (solver-stork.h:163-267): the Chebyshev recurrence over the
 * degree, then the 4-stage finishing blend; returns 1 when out is finite */
static int rock4_substep(float * out, const float * xt, const float * vt, int s, float t_curr, float t_prev, int order,
                         const float * dv, const float * d2v, int64_t n, const orc_rock4 * tab, int * mdeg_out) {
    const int smax = tab->ms[tab->ms_len - 1];
    if (s > smax) {
        s = smax;
    }
    int mdeg, mz, mr;
    rock4_mdegr(s, tab->ms, tab->ms_len, &mdeg, &mz, &mr);
    *mdeg_out      = mdeg;
    const float dt = t_curr - t_prev;
    const size_t b = (size_t) n * sizeof(float) + 4;
    float *      y2 = (float *) malloc(b), *y1 = (float *) malloc(b), *yj = (float *) malloc(b);
    float *      va = (float *) malloc(b), *f1 = (float *) malloc(b), *f2 = (float *) malloc(b);
    float *      f3 = (float *) malloc(b), *f4 = (float *) malloc(b);
    memcpy(y2, xt, (size_t) n * sizeof(float));
    memcpy(y1, xt, (size_t) n * sizeof(float));
    float ci1 = t_curr, ci2 = t_curr, ci3 = t_curr;
    for (int j = 1; j <= mdeg; j++) {
        if (j == 1) {
            const float t1 = -dt * (float) tab->recf[mr];
            ci1            = t_curr + t1;
            ci2            = ci1;
            for (int64_t i = 0; i < n; i++) {
                y1[i] = xt[i] + t1 * vt[i];
            }
        } else {
            const float diff = ci1 - t_curr;
            stork_taylor(va, order, diff, vt, dv, d2v, n);
            const float t1     = -dt * (float) tab->recf[mr + 2 * (j - 2) + 1];
            const float t3     = -(float) tab->recf[mr + 2 * (j - 2) + 2];
            const float t2     = 1.0f - t3;
            const float ci1_nw = t1 + t2 * ci2 + t3 * ci3;
            for (int64_t i = 0; i < n; i++) {
                yj[i] = t1 * va[i] + t2 * y1[i] + t3 * y2[i];
            }
            float * r = y2;
            y2        = y1;
            y1        = yj;
            yj        = r;
            ci3       = ci2;
            ci2       = ci1_nw;
            ci1       = ci1_nw;
        }
    }
    const double * fa = tab->fpa + 6 * mz;
    const double * fb = tab->fpb + 4 * mz;
    const float    a0 = -dt * (float) fa[0];
    stork_taylor(f1, order, ci1 - t_curr, vt, dv, d2v, n);
    float       c2f = ci1 + a0;
    const float a1 = -dt * (float) fa[1], a2 = -dt * (float) fa[2];
    stork_taylor(f2, order, c2f - t_curr, vt, dv, d2v, n);
    c2f            = ci1 + a1 + a2;
    const float a3 = -dt * (float) fa[3], a4 = -dt * (float) fa[4], a5 = -dt * (float) fa[5];
    stork_taylor(f3, order, c2f - t_curr, vt, dv, d2v, n);
    c2f            = ci1 + a3 + a4 + a5;
    const float b0 = -dt * (float) fb[0], b1 = -dt * (float) fb[1], b2 = -dt * (float) fb[2], b3 = -dt * (float) fb[3];
    stork_taylor(f4, order, c2f - t_curr, vt, dv, d2v, n);
    for (int64_t i = 0; i < n; i++) {
        out[i] = y1[i] + b0 * f1[i] + b1 * f2[i] + b2 * f3[i] + b3 * f4[i];
    }
    free(y2), free(y1), free(yj), free(va), free(f1), free(f2), free(f3), free(f4);
    return all_finite(out, n);
}

/* solver_stork4_step (solver-stork.h:269-323). prev/prev2 hold the two most
 * recent velocity records with step sizes h1/h2 (hist = records stored); they
 * are rotated (prev2 <- prev, prev <- vt) as _stork_update_history appends.
 * info[0] = derivative order, info[1] = degree of the accepted sub-stepping
 * (0: Euler), info[2] = 1 when every attempt was non-finite (Euler fallback). */
void orc_stork4_step(float * xt, const float * vt, int64_t n, float t_curr, float t_next, int hist, float h1,
                     float h2, float * prev, float * prev2, int substeps, const orc_rock4 * tab, int * info) {
    const float dt = t_curr - t_next;
    info[0] = info[1] = info[2] = 0;
    if (hist == 0) {
        for (int64_t i = 0; i < n; i++) {
            xt[i] -= vt[i] * dt;
        }
    } else {
        const size_t b   = (size_t) n * sizeof(float) + 4;
        float *      dv  = (float *) calloc(1, b);
        float *      d2v = (float *) calloc(1, b);
        float *      nxt = (float *) malloc(b);
        const int    ord = stork_derivatives(vt, n, hist, prev, h1, prev2, h2, dv, d2v);
        int          s   = substeps >= 2 ? substeps : 2, ok = 0, mdeg = 0;
        while (s >= 2) {
            if (rock4_substep(nxt, xt, vt, s, t_curr, t_next, ord, dv, d2v, n, tab, &mdeg)) {
                ok = 1;
                break;
            }
            s /= 2;
        }
        info[0] = ord;
        if (ok) {
            memcpy(xt, nxt, (size_t) n * sizeof(float));
            info[1] = mdeg;
        } else {
            for (int64_t i = 0; i < n; i++) {
                xt[i] -= vt[i] * dt;
            }
            info[2] = 1;
        }
        free(dv), free(d2v), free(nxt);
    }
    if (hist >= 1) {
        memcpy(prev2, prev, (size_t) n * sizeof(float));
    }
    memcpy(prev, vt, (size_t) n * sizeof(float));
}

/* DCW (dit-sampler.h:626-664): per sample, denoised = xt - vt * t_next, then
 * the Haar band correction of dwt-haar.h (forward 27-52, inverse 56-77, low
 * 84-101, high 105-122, double 127-152, pix 157-166). mode 0 low, 1 high,
 * 2 double, 3 pix; the effective scalers follow dit-sampler.h:641-644. */
static void haar_fwd(const float * src, int64_t t, int64_t c, float * lo, float * hi) {
    const float k = 0.70710678118654752440f;
    for (int64_t l = 0; l < (t + 1) / 2; l++) {
        const float * a = src + 2 * l * c;
        if (2 * l + 1 < t) {
            const float * b = a + c;
            for (int64_t j = 0; j < c; j++) {
                lo[l * c + j] = (a[j] + b[j]) * k;
                hi[l * c + j] = (a[j] - b[j]) * k;
            }
        } else {
            for (int64_t j = 0; j < c; j++) {
                lo[l * c + j] = a[j] * k;
                hi[l * c + j] = a[j] * k;
            }
        }
    }
}

static void haar_inv(const float * lo, const float * hi, int64_t t, int64_t c, float * out) {
    const float k = 0.70710678118654752440f;
    for (int64_t l = 0; l < (t + 1) / 2; l++) {
        for (int64_t j = 0; j < c; j++) {
            out[2 * l * c + j] = (lo[l * c + j] + hi[l * c + j]) * k;
        }
        if (2 * l + 1 < t) {
            for (int64_t j = 0; j < c; j++) {
                out[(2 * l + 1) * c + j] = (lo[l * c + j] - hi[l * c + j]) * k;
            }
        }
    }
}

void orc_dcw(int mode, float * xt, const float * vt, int64_t n, int64_t t, int64_t oc, float t_curr, float t_next,
             float scaler, float high_scaler) {
    const float s_low = t_curr * scaler, s_high = (1.0f - t_curr) * scaler;
    const float s_dh = (1.0f - t_curr) * high_scaler, s_pix = scaler;
    const int64_t m  = t * oc, tl = (t + 1) / 2;
    const size_t  b  = (size_t) (tl * oc) * sizeof(float) + 4;
    float *       den = (float *) malloc((size_t) m * sizeof(float) + 4);
    float *       xl = (float *) malloc(b), *xh = (float *) malloc(b), *yl = (float *) malloc(b),
            *yh = (float *) malloc(b);
    for (int64_t s = 0; s < n; s++) {
        float *       x = xt + s * m;
        const float * v = vt + s * m;
        for (int64_t i = 0; i < m; i++) {
            den[i] = x[i] - v[i] * t_next;
        }
        if (mode == 3) {
            if (s_pix != 0.0f) {
                for (int64_t i = 0; i < m; i++) {
                    x[i] = x[i] + s_pix * (x[i] - den[i]);
                }
            }
            continue;
        }
        const float lo_s = mode == 0 || mode == 2 ? s_low : 0.0f;
        const float hi_s = mode == 1 ? s_high : mode == 2 ? s_dh : 0.0f;
        if (lo_s == 0.0f && hi_s == 0.0f) {
            continue;
        }
        haar_fwd(x, t, oc, xl, xh);
        haar_fwd(den, t, oc, yl, yh);
        if (lo_s != 0.0f) {
            for (int64_t i = 0; i < tl * oc; i++) {
                xl[i] = xl[i] + lo_s * (xl[i] - yl[i]);
            }
        }
        if (hi_s != 0.0f) {
            for (int64_t i = 0; i < tl * oc; i++) {
                xh[i] = xh[i] + hi_s * (xh[i] - yh[i]);
            }
        }
        haar_inv(xl, xh, t, oc, x);
    }
    free(den), free(xl), free(xh), free(yl), free(yh);
}
