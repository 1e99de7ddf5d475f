// launch.h -- host-side launchers shared between the kernel files and the
// C-ABI layer. Arguments reaching these functions have been validated.
#pragma once

#include "common.h"

namespace mi {

// ---- vector helpers ------------------------------------------------------
template <int TO, int N> __device__ __forceinline__ void store_vec(char * p, const float * f) {
    if constexpr (TO == MI_TYPE_F32) {
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            st16(p + 16 * i, pack16<MI_TYPE_F32>(f + 4 * i));
        }
    } else if constexpr (N == 8) {
        st16(p, pack16<TO>(f));
    } else {
        static_assert(N == 4, "4 or 8 half-width elements per store");
        uint2 v;
        if constexpr (TO == MI_TYPE_BF16) {
            v = make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
        } else {
            v = make_uint2(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]));
        }
        st8(p, v);
    }
}

// ---- norm.hip --------------------------------------------------------------
// mode 0: rms_norm; 1: rms_norm * w; 2: (rms_norm * w) * (sc + 1) + sh.
// With `add`, the normalized row is the residual sum x + x2 (* gate),
// optionally clamped, which is also stored to add->ysum.
struct AddNorm {
    const mi_tensor * x2;
    const float *     gate;
    int               clamp;
    float             lo, hi;
    const mi_tensor * ysum;
};

// Head-sized rows (ne0 = 64/128/256) of a row-uniform view, same type in and
// out, 16-byte aligned: RMSNorm (* w) by whole rows per lane group.
// MI_ERR_UNSUPPORTED for any other view (the caller takes another kernel).
int launch_rms_norm_short(const mi_tensor & x, const float * w, float eps, const mi_tensor & y, hipStream_t s);
int launch_rms_norm(const mi_tensor & x, const float * w, const float * sc, const float * sh, float eps,
                    const mi_tensor & y, hipStream_t s, const AddNorm * add = nullptr);

// ---- rope.hip --------------------------------------------------------------
struct HeadSeg {
    const char * x;
    char *       y;
    uint32_t     heads;
    int64_t      xs1, xs2, xs3, ys1, ys2, ys3;
    const float * w;
};

struct HeadArgs {
    HeadSeg         seg[2];
    int             nseg;
    uint32_t        ntok;  // ne2 * ne3
    uint32_t        ne2;
    FastDiv         dne2;
    const int32_t * pos;   // nullptr: no rope
    float           theta_scale, freq_scale, mscale, eps;
    int             ne0, n_dims;
    int             norm;  // apply rms_norm (* w when seg.w)
};

// q and (optionally) k share positions and head size. Returns mi_status.
int launch_heads(HeadArgs & a, int tin, int tout, hipStream_t s);

// QK-norm -> rope of seg[0] (Q, to its y) and seg[1] (K), and V, with K and V
// written into KV caches: flat token t (i2 + i3 * ne2) belongs to sequence
// b = t / T at slot pos0[b] + t % T of cache set sets[b] (b when sets is null).
struct HeadKV {
    const char *    v;             // V rows [D, Nkv, ne2, ne3] (activation type)
    int64_t         vs1, vs2, vs3;
    char *          kc;            // caches [D, max_seq, Nkv, n_sets], one type
    char *          vc;
    int64_t         cnb1, cnb2, cnb3;
    int64_t         max_seq, n_sets;
    const int32_t * pos0;
    const int32_t * sets;
    uint32_t        T;             // tokens per sequence
    FastDiv         dT;
    int             clamp_v;       // V clamped to [-65504, 65504] before the cache cast
    int32_t *       d_err;         // invalid slots or sets, counted per K and V row
};
// MI_ERR_UNSUPPORTED when the shapes or alignments are not the fused kernel's
// (D in {64, 128, 256} rotated whole, 16-byte aligned rows, same in/out type).
int launch_heads_kv(HeadArgs & a, const HeadKV & kv, int tin, int tcache, int rounding, hipStream_t s);

// ---- glu.hip ---------------------------------------------------------------
int launch_swiglu(const char * g, const char * u, int64_t gs, int64_t us, int tin, char * y, int64_t ys, int tout,
                  int64_t rows, int64_t n, bool vec_ok, hipStream_t s);

// ---- binary.hip ------------------------------------------------------------
enum BinOp { OP_ADD = 0, OP_MUL = 1, OP_GATED = 2, OP_MOD = 3, OP_NONE = 4 };

// y = op(a, b | v0, v1), then optional clamp. b is a full tensor of a's shape
// (brow) or nullptr; v0/v1 are F32 [ne0] column vectors.
int launch_binary(int op, const mi_tensor & a, const mi_tensor * b, const float * v0, const float * v1, bool clamp,
                  float lo, float hi, const mi_tensor & y, hipStream_t s);

// generic ggml_can_repeat broadcast (any b shape)
int launch_binary_bcast(int op, const mi_tensor & a, const mi_tensor & b, bool clamp, float lo, float hi,
                        const mi_tensor & y, hipStream_t s);

// ---- getrows.hip -----------------------------------------------------------
int launch_get_rows(const mi_tensor & table, const int32_t * ids, int64_t n_ids, int64_t ids_stride,
                    const mi_tensor & y, int32_t * d_err, hipStream_t s);

// ---- quant.hip -------------------------------------------------------------
// Rows of src [ne0, ne1, ne2, ne3] copied/converted into dst rows. Row r of
// src = (i1, i2, i3); dst row address:
//   plain cpy : dst + i1*nb1 + i2*nb2 + i3*nb3
//   kv store  : cache + (pos0[i3] + i2)*nb1 + i1*nb2 + set[i3]*nb3
struct RowCopy {
    const char *    src;
    Rows3           sr;
    uint32_t        rows;
    int             ne0;
    char *          dst;
    Rows3           dr;         // plain cpy
    // kv store
    int             kv;
    uint32_t        ne1, ne2;   // src heads, tokens per sequence
    FastDiv         d1, d2;
    const int32_t * pos0;
    const int32_t * sets;
    int64_t         cnb1, cnb2, cnb3;
    int64_t         max_seq, n_sets;
    int32_t *       d_err;
};

int launch_row_copy(const RowCopy & k, const RowCopy * v, int tin, int tout, int rounding, hipStream_t s);

// ---- fattn.hip -------------------------------------------------------------
// ggml_flash_attn_ext operands (byte strides; ne0 = D contiguous everywhere)
struct FaArgs {
    const char * q;  // [D, n_q, Nh, N]: q1 = position, q2 = head, q3 = batch
    int64_t      q1, q2, q3;
    int          tq;
    int          qvec;  // q rows 16-byte aligned (base and q1/q2/q3 strides)
    const char * k;  // [D, n_kv, Nkv, N / rk3]
    int64_t      k1, k2, k3;
    const char * v;
    int64_t      v1, v2, v3;
    const char * mask;  // F16 [n_kv, >= n_q, mne2, mne3] or nullptr
    int64_t      m1, m2, m3;
    int          mne2, mne3;
    int          mshared;  // every row of a wave uses one mask row (set by flash_attn_plan)
    int          mfma;     // the matrix-core prefill path (set by flash_attn_plan)
    int          dec;      // the matrix-core decode kernel (set by flash_attn_plan)
    int          yvec;     // y rows 16-byte aligned
    int          mvec;     // mask rows 8-byte aligned (4 fp16 per load)
    int          ngq;      // matrix-core path: groups of 16 query positions in the mask summary
    uint8_t *    msum;     // matrix-core path with a mask: per (mask batch, mask head, group, key tile)
                           // bit 0 = some key not -inf, bit 1 = some value not 0 (in the workspace)
    char *       y;  // F32 [D, Nh, n_q, N]: y1 = head, y2 = position, y3 = batch
    int64_t      y1, y2, y3;
    int          n_q, n_kv, nh, nkv, nb, rk, rk3;
    int          kt;  // K and V type
    float        scale;
    int          rows, rblocks, chunk, splits;  // from flash_attn_plan
    float *      ws;                            // split partials (flash_attn_workspace bytes)
    // matrix-core path: row blocks of 128 per (sequence, KV head); work items
    // [0, tfull) whole, the next tsplit as two halves of the key tiles (tiles
    // [0, tmid) and [tmid, end)) whose partials go to fpart
    int          rblk, tfull, tsplit, tmid;
    float *      fpart;
};

void   flash_attn_plan(FaArgs & a, int D);
size_t flash_attn_workspace(const FaArgs & a, int D);
size_t flash_attn_part_offset(const FaArgs & a);
int    launch_flash_attn(const FaArgs & a, int kt, int D, hipStream_t s);

// ---- matmul.hip ------------------------------------------------------------
// ggml_mul_mat(w, x), Q8_0 weights in the R64 layout, F32 x rows
struct MmvArgs {
    const char * w;       // R64 weights: quants, then scales at w + qbytes
    uint64_t     qbytes;  // ng * nbk * 2048
    uint32_t     k, n, nbk, ng, npad;  // K, N (weight rows), K / 32, row groups of 64, 64 * ng
    const char * x;       // F32 x rows: element i of row m at x + m * x1 + 4 i
    int64_t      x1;
    int          xvec;    // x rows 16-byte aligned
    uint32_t     m;       // rows of x
    uint32_t     mp;      // row stride of the quantized x (m, or m padded to 128 for the matrix kernel)
    char *       y;       // F32 y: element n of row m at y + m * y1 + 4 n
    int64_t      y1;
    uint32_t     splits, wpg, bps;  // workgroups per row group, waves (key splits) per workgroup,
                                    // blocks per wave (set by mul_mat_q8_0_plan)
    const float * nw;          // non-null: x = rms_norm(x) * nw (the norm prologue), with eps
    float        eps;
    const char * ab;           // non-null (with nw): x = x + ab first, rows at stride ab1,
    int64_t      ab1;          // the sum written to sum (rows at stride sum1)
    const float * gate;        // non-null (with ab): x = x + ab * gate (the DiT's gated residual)
    const float * msc;         // non-null (with nw): the normalized rows modulated,
    const float * msh;         // (x' * (msc + 1)) + msh (the DiT's AdaLN)
    char *       sum;
    int64_t      sum1;
    int          glu;          // 1: x = silu(g) * u (the SwiGLU prologue), rows at stride gu1
    const char * g;
    const char * u;
    int64_t      gu1;
    const char * res;          // non-null: y = y + res (ggml_add after the product), rows at stride res1,
    int64_t      res1;         // then clamped to [rlo, rhi] when rclamp (ggml_clamp)
    int          rclamp;
    float        rlo, rhi;
    const float * rgate;       // non-null (with res): y = res + y * rgate[n] (the DiT's gated residual)
    char *       xq;           // workspace: quantized x [m][k]
    float *      xd;           //            scales [m][nbk]
    float *      part;         //            partials [splits][m][npad] (splits > 1)
};

void   mul_mat_q8_0_plan(MmvArgs & a, int cus);
size_t mul_mat_q8_0_workspace(const MmvArgs & a);
void   mul_mat_q8_0_bind(MmvArgs & a, char * ws);
int    launch_mul_mat_q8_0(const MmvArgs & a, hipStream_t s);
int    launch_q8_0_repack(const char * src, int64_t nb1, uint32_t k, uint32_t n, char * dst, hipStream_t s);

// ---- sampler.hip -----------------------------------------------------------
struct ApgArgs {
    const float * cond;    // F32 [n][t][oc]
    const float * uncond;
    double *      ra;      // momentum running average [n][t][oc] (kept across steps)
    float *       out;
    uint32_t      n, t, oc;
    int           first;   // the buffer is uninitialized: ra = diff
    float         scale, threshold;
    double        momentum;
};
struct FlowArgs {
    float *       xt;      // updated in place (euler, dpm3m)
    const float * vt;
    float *       prev;    // dpm3m history (updated in place)
    float *       prev2;
    float *       out;     // final step
    const float * noise;   // sde: the step's N(0,1) draws
    uint64_t      n;
    int           solver;  // 0 euler, 1 dpm3m, 2 final, 3 sde
    int           hist;    // dpm3m: stored velocities (0, 1, 2)
    float         t_curr, t_next;
};
int launch_apg(const ApgArgs & a, hipStream_t s);
int launch_flow_step(const FlowArgs & a, hipStream_t s);

// STORK4: one step is a statistics pass (the derivative guards' sums of
// squares), one launch per sub-stepping attempt (halving degrees), and a commit
// pass. The fp32 scalar chains of each attempt are computed on the host in the
// reference's order and travel in the attempt's kernel arguments.
constexpr int STORK_MAX_DEG      = 160;  // largest ROCK4 degree accepted
constexpr int STORK_MAX_ATTEMPTS = 16;
constexpr int STORK_STAT_BLOCKS  = 256;
struct StorkPlan {
    float   t1_first;                  // j = 1: -dt * recf[mr]
    float   fin_diff[4];               // time offsets of the four finishing velocities
    float   fpb[4];                    // -dt * fpb[mz][k]
    int32_t mdeg;
    int32_t attempt;                   // index in the step's attempt list
    float   sub[STORK_MAX_DEG - 1][4]; // j = 2..mdeg: temp1, temp2, temp3, diff
};
struct StorkArgs {
    float *       xt;          // updated in place by the commit pass
    const float * vt;
    float *       prev;        // latest stored velocity (step size h1), rotated by the commit
    float *       prev2;       // the one before (h2)
    uint32_t *    status;      // workspace: [0] Euler fallbacks this generation, [1] derivative
                               // order, [2] accepted degree, [4..4+STORK_MAX_ATTEMPTS) non-finite flags
    double *      part;        // workspace: [STORK_STAT_BLOCKS][3] sums of squares (vt, dv, d2v)
    float *       xnext;       // workspace: [n] the latest attempt's result
    uint64_t      n;
    int           hist;        // stored velocities (0: Euler bootstrap)
    int           max_order;   // derivative order the step sizes allow (0, 1, 2)
    float         h1, h2, dt;
    double        c2;          // 2 / (h1 h2 (h1 + h2)) for d2v
    int           n_attempts;
    int32_t       att_deg[STORK_MAX_ATTEMPTS];
};
constexpr size_t STORK_WS_STATUS = 256;
constexpr size_t STORK_WS_XNEXT  = STORK_WS_STATUS + ((STORK_STAT_BLOCKS * 3 * sizeof(double) + 255) / 256) * 256;
int launch_stork4(const StorkArgs & a, const StorkPlan * plans, hipStream_t s);

// DCW: Haar band correction after a solver step, per frame pair and channel.
struct DcwArgs {
    float *       xt;      // [n][t][oc], in place
    const float * vt;
    uint32_t      n, t, oc;
    float         t_next;
    float         lo_s, hi_s;  // band scalers (0: band untouched)
    int           pix;         // pixel-space mode: xt += lo_s (xt - denoised)
};
int launch_dcw(const DcwArgs & a, hipStream_t s);

// ---- tsembd.hip ------------------------------------------------------------
int launch_scale(const mi_tensor & x, float sc, const mi_tensor & y, hipStream_t s);
int launch_timestep_embedding(const float * t, int64_t n, int64_t ts, int dim, int max_period, char * y,
                              int64_t ys, hipStream_t s);

}  // namespace mi
