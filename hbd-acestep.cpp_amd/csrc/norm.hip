// norm.hip -- RMSNorm over long rows (hidden size), optionally fused with the
// weight multiply and the DiT AdaLN modulate.
//
// ggml node chain reproduced (reference: qwen3-enc.h:114-120,
// dit-graph.h:24-30 and 54-64):
//   n = rms_norm(x, eps)          sum_i (double)(x_i*x_i); mean = (float)(sum/ne0);
//                                 scale = 1.0f/sqrtf(mean + eps); n_i = x_i*scale
//                                 (F32 rows; BF16/F16 rows sum the squares in fp32)
//   n = n * w                     (ggml_mul, [ne0] broadcast)
//   m = (n * (scale_v + 1)) + shift_v   (dit_ggml_adaln)
// Every intermediate stays fp32 in registers, rounded exactly as the ggml
// nodes round it; only the final value is converted to the output type.
//
// Fast path: one workgroup owns whole rows. Each thread always handles the
// same C 16-byte column vectors, so the F32 weight / (scale+1) / shift
// vectors are loaded once into registers and reused for every row the
// workgroup processes. R rows are loaded before any is reduced so each lane
// keeps R*C 128-bit loads in flight; per-row partial sums (double for F32
// rows, fp32 for 16-bit rows) are reduced in-wave with DPP, then across waves
// through LDS in a fixed order.
#include "launch.h"

namespace mi {

struct NormArgs {
    const char *  x;
    char *        y;
    Rows3         xr, yr;
    uint32_t      rows;
    int           n;
    float         eps;
    const float * w;
    const float * sc;
    const float * sh;
    // fused residual add in front of the norm (ADD != 0):
    //   v = x + x2 (ADD 1), x + x2 * gate (ADD 2), clamp(x + x2) (ADD 3);
    //   v is stored (ysum, rounded to the activation type) and normalized.
    const char *  x2;
    Rows3         x2r;
    char *        ysum;
    Rows3         ysr;
    const float * gate;
    int           clamp;
    float         lo, hi;
};

#ifndef MI_NORM_R
#define MI_NORM_R 4  // rows per workgroup iteration when each thread owns one vector
#endif


template <int TI, int TO, int MODE, int ADD, int C, int R>
__global__ void __launch_bounds__(512) k_rms_rows(const NormArgs a) {
    constexpr int VI = TT<TI>::VEC;
    constexpr int EI = TT<TI>::ES;
    constexpr int EO = TT<TO>::ES;
    const int     T    = blockDim.x;
    const int     tid  = threadIdx.x;
    const int     wave = tid >> 6;
    const int     lane = tid & 63;
    const int     nw   = T >> 6;

    using acc_t = sq_t<TI>;
    __shared__ acc_t part[2][R][8];

    float wv[C][VI], sv[C][VI], hv[C][VI], gv[C][VI];
    if constexpr (ADD == 2) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int col = (j * T + tid) * VI;
#pragma unroll
            for (int e = 0; e < VI; e += 4) {
                const float4 g4 = *(const float4 *) (a.gate + col + e);
                gv[j][e + 0]    = g4.x;
                gv[j][e + 1]    = g4.y;
                gv[j][e + 2]    = g4.z;
                gv[j][e + 3]    = g4.w;
            }
        }
    }
    if constexpr (MODE >= 1) {
#pragma unroll
        for (int j = 0; j < C; ++j) {
            const int col = (j * T + tid) * VI;
#pragma unroll
            for (int e = 0; e < VI; e += 4) {
                const float4 w4 = *(const float4 *) (a.w + col + e);
                wv[j][e + 0]    = w4.x;
                wv[j][e + 1]    = w4.y;
                wv[j][e + 2]    = w4.z;
                wv[j][e + 3]    = w4.w;
                if constexpr (MODE == 2) {
                    const float4 s4 = *(const float4 *) (a.sc + col + e);
                    const float4 h4 = *(const float4 *) (a.sh + col + e);
                    sv[j][e + 0]    = s4.x + 1.0f;
                    sv[j][e + 1]    = s4.y + 1.0f;
                    sv[j][e + 2]    = s4.z + 1.0f;
                    sv[j][e + 3]    = s4.w + 1.0f;
                    hv[j][e + 0]    = h4.x;
                    hv[j][e + 1]    = h4.y;
                    hv[j][e + 2]    = h4.z;
                    hv[j][e + 3]    = h4.w;
                }
            }
        }
    }

    int it = 0;
    for (uint32_t rbase = blockIdx.x * R; rbase < a.rows; rbase += gridDim.x * R, ++it) {
        uint4 raw[R][C], raw2[ADD ? R : 1][ADD ? C : 1];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = rbase + r;
            if (row < a.rows) {
                const char * xp  = a.x + (int64_t) row * a.xr.s1;
                const char * x2p = ADD ? a.x2 + (int64_t) row * a.x2r.s1 : nullptr;
#pragma unroll
                for (int j = 0; j < C; ++j) {
                    raw[r][j] = ld16(xp + (size_t) ((j * T + tid) * VI) * EI);
                    if constexpr (ADD != 0) {
                        raw2[r][j] = ld16(x2p + (size_t) ((j * T + tid) * VI) * EI);
                    }
                }
            } else {
#pragma unroll
                for (int j = 0; j < C; ++j) {
                    raw[r][j] = make_uint4(0, 0, 0, 0);
                    if constexpr (ADD != 0) {
                        raw2[r][j] = make_uint4(0, 0, 0, 0);
                    }
                }
            }
        }
        // residual add (ggml_add / dit_ggml_gated_add, then ggml_clamp); the
        // sum is rounded to the activation type first, exactly as the unfused
        // add kernel would store it and the norm kernel read it back
        float xin[R][C][VI];
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < C; ++j) {
                unpack16<TI>(raw[r][j], xin[r][j]);
                if constexpr (ADD != 0) {
                    float f2[VI];
                    unpack16<TI>(raw2[r][j], f2);
#pragma unroll
                    for (int e = 0; e < VI; ++e) {
                        float v;
                        if constexpr (ADD == 2) {
                            const float gx = f2[e] * gv[j][e];
                            v              = xin[r][j][e] + gx;
                        } else {
                            v = xin[r][j][e] + f2[e];
                        }
                        if constexpr (ADD == 3) {
                            const float c = v < a.hi ? v : a.hi;
                            v             = c > a.lo ? c : a.lo;
                        }
                        xin[r][j][e] = round_to<TO>(v);
                    }
                }
            }
        }
        if constexpr (ADD != 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const uint32_t row = rbase + r;
                if (row < a.rows) {
                    char * sp = a.ysum + (int64_t) row * a.ysr.s1;
#pragma unroll
                    for (int j = 0; j < C; ++j) {
                        store_vec<TO, VI>(sp + (size_t) ((j * T + tid) * VI) * EO, xin[r][j]);
                    }
                }
            }
        }
        acc_t s[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            s[r] = 0;
#pragma unroll
            for (int j = 0; j < C; ++j) {
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    s[r] = sq_acc<TI>(s[r], xin[r][j][e]);
                }
            }
            s[r] = group_sum<64>(s[r]);
        }
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                part[it & 1][r][wave] = s[r];
            }
        }
        __syncthreads();
        // the R row scales in one pass (each costs ~40 instructions, the same
        // for one lane as for all 64): lane r sums row r's wave partials, in
        // wave order, and computes its scale; row r then reads lane r
        float scl;
        {
            const int rr  = lane < R ? lane : 0;
            acc_t     tot = 0;
            for (int q = 0; q < nw; ++q) {
                tot += part[it & 1][rr][q];
            }
            scl = rms_scale(tot, a.n, a.eps);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = rbase + r;
            if (row >= a.rows) {
                continue;
            }
            const float scale = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(scl), r));
            char *      yp    = a.y + (int64_t) row * a.yr.s1;
#pragma unroll
            for (int j = 0; j < C; ++j) {
                float f[VI];
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    float v = xin[r][j][e] * scale;
                    if constexpr (MODE >= 1) {
                        v = v * wv[j][e];
                    }
                    if constexpr (MODE == 2) {
                        v = v * sv[j][e];
                        v = v + hv[j][e];
                    }
                    f[e] = v;
                }
                store_vec<TO, VI>(yp + (size_t) ((j * T + tid) * VI) * EO, f);
            }
        }
    }
}

template <int TI, int TO, int MODE>
__global__ void __launch_bounds__(256) k_rms_rows_generic(const NormArgs a) {
    constexpr int EI    = TT<TI>::ES;
    constexpr int EO    = TT<TO>::ES;
    const int     lane  = threadIdx.x & 63;
    const int     wpb   = blockDim.x >> 6;
    for (uint32_t row = blockIdx.x * wpb + (threadIdx.x >> 6); row < a.rows; row += gridDim.x * wpb) {
        const char * xp  = a.x + a.xr.off(row);
        const char * x2p = a.x2 ? a.x2 + a.x2r.off(row) : nullptr;
        char *       sp  = a.x2 ? a.ysum + a.ysr.off(row) : nullptr;
        char *       yp  = a.y + a.yr.off(row);
        // input of the norm: x, or the (clamped) residual sum rounded to the
        // activation type as it is stored
        auto xval = [&](int i) {
            float v = load_elem<TI>(xp + (size_t) i * EI);
            if (x2p) {
                const float f2 = load_elem<TI>(x2p + (size_t) i * EI);
                if (a.gate) {
                    const float gx = f2 * a.gate[i];
                    v              = v + gx;
                } else {
                    v = v + f2;
                }
                if (a.clamp) {
                    const float c = v < a.hi ? v : a.hi;
                    v             = c > a.lo ? c : a.lo;
                }
                v = round_to<TO>(v);
            }
            return v;
        };
        sq_t<TI> s = 0;  // the fast kernels' accumulator: double for F32 rows, fp32 fma for BF16/F16
        for (int i = lane; i < a.n; i += 64) {
            const float f = xval(i);
            if (sp) {
                store_elem<TO>(sp + (size_t) i * EO, f);
            }
            s = sq_acc<TI>(s, f);
        }
        s                 = group_sum<64>(s);
        const float scale = rms_scale(s, a.n, a.eps);
        for (int i = lane; i < a.n; i += 64) {
            // with a fused add, read back this lane's stored sum (ysum may
            // alias the residual input, so the sum is not recomputed)
            float v = (sp ? load_elem<TO>(sp + (size_t) i * EO) : load_elem<TI>(xp + (size_t) i * EI)) * scale;
            if constexpr (MODE >= 1) {
                v = v * a.w[i];
            }
            if constexpr (MODE == 2) {
                v = v * (a.sc[i] + 1.0f);
                v = v + a.sh[i];
            }
            store_elem<TO>(yp + (size_t) i * EO, v);
        }
    }
}

#ifndef MI_NORM_WPC
#define MI_NORM_WPC 16  // resident waves per CU the grid is sized for
#endif

// Head-sized rows (D = 64, 128 or 256 elements) of a row-uniform view, RMSNorm
// (* w), nothing else: the per-head Q/K norm with no rope (cross attention).
// A row spans L = D/VI lanes, one 16-byte vector each, so one load instruction
// of a wave covers 64/L whole consecutive rows (1 KB); each wave issues U of
// them (U*64/L rows) before it reduces any, and walks such chunks with a
// stride over a grid balanced so that every wave takes the same number of
// chunks (+-1). The row sums are DPP group sums within the L lanes.
//
// Rows past the end of the view load and store the last row again (the same
// values to the same bytes), so no load or store sits behind a branch.
template <int TI, int D, bool W, int U>
__global__ void __launch_bounds__(256) k_rms_short(const char * x, char * y, int64_t xs, int64_t ys, uint32_t rows,
                                                   const float * w, float eps) {
    constexpr int VI  = TT<TI>::VEC;
    constexpr int L   = D / VI;   // lanes per row
    constexpr int RPI = 64 / L;   // rows per load instruction
    constexpr int CH  = U * RPI;  // rows per chunk
    const int     lane = threadIdx.x & 63;
    const int     j    = lane % L;
    const int     g    = lane / L;
    float         wl[VI];
#pragma unroll
    for (int e = 0; e < VI; ++e) {
        wl[e] = W ? w[j * VI + e] : 1.0f;
    }
    // rows < 2^31 (the entry point's bound) and the stride is far below 2^31,
    // so the 32-bit row indices do not wrap
    const uint32_t step = gridDim.x * 4 * CH;
    for (uint32_t base = (blockIdx.x * 4 + (threadIdx.x >> 6)) * CH; base < rows; base += step) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint32_t r = base + u * RPI + g;
            r          = r < rows ? r : rows - 1;
            v[u]       = ld16(x + (int64_t) r * xs + j * 16);
        }
        __builtin_amdgcn_sched_barrier(0);  // all U loads issued before the first is used
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float f[VI];
            unpack16<TI>(v[u], f);
            sq_t<TI> ss = 0;
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                ss = sq_acc<TI>(ss, f[e]);
            }
            ss                = group_sum<L>(ss);
            const float scale = rms_scale(ss, D, eps);
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                f[e] = W ? f[e] * scale * wl[e] : f[e] * scale;
            }
            uint32_t r = base + u * RPI + g;
            r          = r < rows ? r : rows - 1;
            store_vec<TI, VI>(y + (int64_t) r * ys + j * 16, f);
        }
    }
}

#ifndef MI_SHORT_U
#define MI_SHORT_U 4  // load instructions per wave in flight
#endif

template <int TI, int D>
static void launch_short_d(const char * x, char * y, int64_t xs, int64_t ys, uint32_t rows, const float * w, float eps,
                           hipStream_t s) {
    constexpr int  RPI    = 64 / (D / TT<TI>::VEC);
    const uint64_t chunks = ((uint64_t) rows + MI_SHORT_U * RPI - 1) / (MI_SHORT_U * RPI);
    const uint64_t maxw   = (uint64_t) num_cus() * MI_NORM_WPC;
    const uint64_t per    = (chunks + maxw - 1) / maxw;
    const uint64_t waves  = (chunks + per - 1) / per;
    const dim3     grid((uint32_t) ((waves + 3) / 4));
    if (w) {
        MI_LAUNCH((k_rms_short<TI, D, true, MI_SHORT_U>), grid, dim3(256), 0, s, x, y, xs, ys, rows, w, eps);
    } else {
        MI_LAUNCH((k_rms_short<TI, D, false, MI_SHORT_U>), grid, dim3(256), 0, s, x, y, xs, ys, rows, w,
                           eps);
    }
}

template <int TI>
static int launch_short_t(const char * x, char * y, int64_t xs, int64_t ys, uint32_t rows, int d, const float * w,
                          float eps, hipStream_t s) {
    switch (d) {
        case 64:
            launch_short_d<TI, 64>(x, y, xs, ys, rows, w, eps, s);
            return MI_OK;
        case 128:
            launch_short_d<TI, 128>(x, y, xs, ys, rows, w, eps, s);
            return MI_OK;
        case 256:
            launch_short_d<TI, 256>(x, y, xs, ys, rows, w, eps, s);
            return MI_OK;
        default:
            return MI_ERR_UNSUPPORTED;
    }
}

int launch_rms_norm_short(const mi_tensor & x, const float * w, float eps, const mi_tensor & y, hipStream_t s) {
    const Rows3 xr = make_rows3(x), yr = make_rows3(y);
    const bool  ok = x.type == y.type && xr.uni && yr.uni && aligned(x.data, 16) && aligned(y.data, 16) &&
                    x.nb[1] % 16 == 0 && y.nb[1] % 16 == 0 && (!w || aligned(w, 16)) &&
                    x.nb[0] == (uint64_t) type_size(x.type) && y.nb[0] == (uint64_t) type_size(y.type);
    if (!ok) {
        return MI_ERR_UNSUPPORTED;
    }
    const uint32_t rows = (uint32_t) nrows(x);
    if (rows == 0) {
        return MI_OK;
    }
    const char * xp = (const char *) x.data;
    char *       yp = (char *) y.data;
    switch (x.type) {
        case MI_TYPE_F32:
            return launch_short_t<MI_TYPE_F32>(xp, yp, x.nb[1], y.nb[1], rows, (int) x.ne[0], w, eps, s);
        case MI_TYPE_BF16:
            return launch_short_t<MI_TYPE_BF16>(xp, yp, x.nb[1], y.nb[1], rows, (int) x.ne[0], w, eps, s);
        case MI_TYPE_F16:
            return launch_short_t<MI_TYPE_F16>(xp, yp, x.nb[1], y.nb[1], rows, (int) x.ne[0], w, eps, s);
        default:
            return MI_ERR_UNSUPPORTED;
    }
}

// Workgroups for a grid-stride loop over ceil(rows/R) row groups, capped at
// about MI_NORM_WPC resident waves per CU, with the groups spread evenly (every
// workgroup runs the same number of iterations, +-1).
#ifndef MI_NORM_MAXW
#define MI_NORM_MAXW 8  // most waves sharing one row (more waves: fewer columns per lane)
#endif


static uint32_t balanced_grid(uint32_t rows, int R, int nw) {
    const uint32_t iters  = (rows + R - 1) / R;
    const uint32_t max_wg = (uint32_t) num_cus() * (uint32_t) (MI_NORM_WPC / nw > 0 ? MI_NORM_WPC / nw : 1);
    const uint32_t per    = (iters + max_wg - 1) / max_wg;
    return (iters + per - 1) / per;
}

template <int TI, int TO, int MODE, int ADD>
static int dispatch_fast_add(const NormArgs & a, int T, int C, hipStream_t s) {
    const int nw = T / 64;
    switch (C) {
        case 1:
            MI_LAUNCH((k_rms_rows<TI, TO, MODE, ADD, 1, MI_NORM_R>),
                               dim3(balanced_grid(a.rows, MI_NORM_R, nw)), dim3(T), 0, s, a);
            break;
        case 2:
            MI_LAUNCH((k_rms_rows<TI, TO, MODE, ADD, 2, 2>), dim3(balanced_grid(a.rows, 2, nw)), dim3(T), 0,
                               s, a);
            break;
        case 3:
            MI_LAUNCH((k_rms_rows<TI, TO, MODE, ADD, 3, 2>), dim3(balanced_grid(a.rows, 2, nw)), dim3(T), 0,
                               s, a);
            break;
        case 4:
            MI_LAUNCH((k_rms_rows<TI, TO, MODE, ADD, 4, 2>), dim3(balanced_grid(a.rows, 2, nw)), dim3(T), 0,
                               s, a);
            break;
        default:
            return MI_ERR_UNSUPPORTED;
    }
    return MI_OK;
}

template <int TI, int TO, int MODE>
static int dispatch_fast(const NormArgs & a, int T, int C, hipStream_t s) {
    if (a.x2 == nullptr) {
        return dispatch_fast_add<TI, TO, MODE, 0>(a, T, C, s);
    }
    if (a.gate != nullptr) {
        return dispatch_fast_add<TI, TO, MODE, 2>(a, T, C, s);
    }
    if (a.clamp) {
        return dispatch_fast_add<TI, TO, MODE, 3>(a, T, C, s);
    }
    return dispatch_fast_add<TI, TO, MODE, 1>(a, T, C, s);
}

template <int TI, int TO>
static int dispatch_types(const NormArgs & a, int mode, bool fast, int T, int C, hipStream_t s) {
    if (fast) {
        switch (mode) {
            case 0:
                return dispatch_fast<TI, TO, 0>(a, T, C, s);
            case 1:
                return dispatch_fast<TI, TO, 1>(a, T, C, s);
            default:
                return dispatch_fast<TI, TO, 2>(a, T, C, s);
        }
    }
    const uint32_t wpb  = 4;
    uint32_t       grid = (a.rows + wpb - 1) / wpb;
    const uint32_t cap  = (uint32_t) num_cus() * 8;
    grid                = grid > cap ? cap : grid;
    switch (mode) {
        case 0:
            MI_LAUNCH((k_rms_rows_generic<TI, TO, 0>), dim3(grid), dim3(256), 0, s, a);
            break;
        case 1:
            MI_LAUNCH((k_rms_rows_generic<TI, TO, 1>), dim3(grid), dim3(256), 0, s, a);
            break;
        default:
            MI_LAUNCH((k_rms_rows_generic<TI, TO, 2>), dim3(grid), dim3(256), 0, s, a);
            break;
    }
    return MI_OK;
}

int launch_rms_norm(const mi_tensor & x, const float * w, const float * sc, const float * sh, float eps,
                    const mi_tensor & y, hipStream_t s, const AddNorm * add) {
    NormArgs a{};
    a.x    = (const char *) x.data;
    a.y    = (char *) y.data;
    a.xr   = make_rows3(x);
    a.yr   = make_rows3(y);
    a.rows = (uint32_t) nrows(x);
    a.n    = (int) x.ne[0];
    a.eps  = eps;
    a.w    = w;
    a.sc   = sc;
    a.sh   = sh;
    if (add) {
        a.x2    = (const char *) add->x2->data;
        a.x2r   = make_rows3(*add->x2);
        a.ysum  = (char *) add->ysum->data;
        a.ysr   = make_rows3(*add->ysum);
        a.gate  = add->gate;
        a.clamp = add->clamp;
        a.lo    = add->lo;
        a.hi    = add->hi;
    }
    if (a.rows == 0 || a.n == 0) {
        return MI_OK;
    }
    const int mode = sh ? 2 : (w ? 1 : 0);

    // fast path: rows split into 64*nw lanes x C vectors of 16 bytes
    bool      fast = x.type == y.type;
    const int VI   = 16 / type_size(x.type);
    int       T = 0, C = 0;
    if (fast && a.n % (64 * VI) == 0) {
        const int k = a.n / (64 * VI);
        int       nw = 1;
        for (int d = MI_NORM_MAXW; d >= 1; --d) {
            if (k % d == 0) {
                nw = d;
                break;
            }
        }
        T = nw * 64;
        C = k / nw;
    }
    fast = fast && C >= 1 && C <= 4;
    for (int d = 0; d < 4 && fast; ++d) {
        if (d > 0 && ((x.nb[d] % 16) || (y.nb[d] % 16))) {
            fast = false;
        }
    }
    fast = fast && aligned(x.data, 16) && aligned(y.data, 16) && (!w || aligned(w, 16)) &&
           (!sc || aligned(sc, 16)) && (!sh || aligned(sh, 16));
    // the fast kernel addresses row r at r * nb1 in every operand
    fast = fast && a.xr.uni && a.yr.uni && (!add || (a.x2r.uni && a.ysr.uni));
    // its fused add is either gated or clamped, not both
    fast = fast && (!add || !(add->gate && add->clamp));
    if (add) {
        fast = fast && add->x2->type == x.type && add->ysum->type == x.type && aligned(add->x2->data, 16) &&
               aligned(add->ysum->data, 16) && (!add->gate || aligned(add->gate, 16));
        for (int d = 1; d < 4 && fast; ++d) {
            fast = add->x2->nb[d] % 16 == 0 && add->ysum->nb[d] % 16 == 0;
        }
    }

    switch (x.type) {
        case MI_TYPE_F32:
            switch (y.type) {
                case MI_TYPE_F32:
                    return dispatch_types<MI_TYPE_F32, MI_TYPE_F32>(a, mode, fast, T, C, s);
                case MI_TYPE_BF16:
                    return dispatch_types<MI_TYPE_F32, MI_TYPE_BF16>(a, mode, false, T, C, s);
                default:
                    return dispatch_types<MI_TYPE_F32, MI_TYPE_F16>(a, mode, false, T, C, s);
            }
        case MI_TYPE_BF16:
            switch (y.type) {
                case MI_TYPE_F32:
                    return dispatch_types<MI_TYPE_BF16, MI_TYPE_F32>(a, mode, false, T, C, s);
                case MI_TYPE_BF16:
                    return dispatch_types<MI_TYPE_BF16, MI_TYPE_BF16>(a, mode, fast, T, C, s);
                default:
                    return dispatch_types<MI_TYPE_BF16, MI_TYPE_F16>(a, mode, false, T, C, s);
            }
        default:
            switch (y.type) {
                case MI_TYPE_F32:
                    return dispatch_types<MI_TYPE_F16, MI_TYPE_F32>(a, mode, false, T, C, s);
                case MI_TYPE_BF16:
                    return dispatch_types<MI_TYPE_F16, MI_TYPE_BF16>(a, mode, false, T, C, s);
                default:
                    return dispatch_types<MI_TYPE_F16, MI_TYPE_F16>(a, mode, fast, T, C, s);
            }
    }
}

}  // namespace mi
