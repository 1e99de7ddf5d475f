// binary.hip -- elementwise ops over rows with [ne0] column vectors:
//   OP_ADD   y = a + b            (ggml_add, same shape)      qwen3-lm.h:479, 730
//            y = a + v0           (ggml_add, [ne0] broadcast)
//   OP_MUL   y = a * b | a * v0   (ggml_mul)
//   OP_GATED y = a + (b * v0)     (dit_ggml_gated_add, dit-graph.h:70-76)
//   OP_MOD   y = (a * (v0 + 1)) + v1   (dit_ggml_adaln, dit-graph.h:54-64)
//   OP_NONE  y = a
// followed, when requested, by ggml_clamp: MAX(MIN(y, hi), lo)
// (qwen3-lm.h:481, 732). Each result is rounded exactly as the separate
// ggml nodes round it.
//
// Fast path: a flat one-shot grid, one (or MI_BIN_U) 16-byte vector per
// thread, the F32 column vectors read through the caches. The row-stationary
// kernel (a workgroup spans whole rows, each thread keeps its column vectors
// in registers) remains for builds with MI_BIN_FLAT=0.
#include "launch.h"

namespace mi {

struct BinArgs {
    const char *  a;
    const char *  b;
    char *        y;
    Rows3         ar, br, yr;
    const float * v0;
    const float * v1;
    uint32_t      rows;
    int           n;
    int           clamp;
    float         lo, hi;
};

template <int OP, bool BROW>
__device__ __forceinline__ float bin_apply(float a, float b, float v0, float v1) {
    if constexpr (OP == OP_ADD) {
        return BROW ? a + b : a + v0;
    } else if constexpr (OP == OP_MUL) {
        return BROW ? a * b : a * v0;
    } else if constexpr (OP == OP_GATED) {
        const float g = b * v0;
        return a + g;
    } else if constexpr (OP == OP_MOD) {
        const float m = a * v0;  // v0 already holds scale + 1
        return m + v1;
    } else {
        return a;
    }
}

template <int T_, int OP, bool BROW, int C, int R>
__global__ void __launch_bounds__(512) k_bin_rows(const BinArgs a) {
    constexpr int VI  = TT<T_>::VEC;
    constexpr int ES  = TT<T_>::ES;
    constexpr bool V0 = (OP == OP_GATED || OP == OP_MOD || ((OP == OP_ADD || OP == OP_MUL) && !BROW));
    constexpr bool V1 = (OP == OP_MOD);
    constexpr bool LB = BROW || OP == OP_GATED;
    const int      T   = blockDim.x;
    const int      tid = threadIdx.x;

    float c0[C][VI], c1[C][VI];
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const int col = (j * T + tid) * VI;
#pragma unroll
        for (int e = 0; e < VI; e += 4) {
            if constexpr (V0) {
                const float4 q = *(const float4 *) (a.v0 + col + e);
                const float  k = OP == OP_MOD ? 1.0f : 0.0f;
                c0[j][e + 0]   = OP == OP_MOD ? q.x + k : q.x;
                c0[j][e + 1]   = OP == OP_MOD ? q.y + k : q.y;
                c0[j][e + 2]   = OP == OP_MOD ? q.z + k : q.z;
                c0[j][e + 3]   = OP == OP_MOD ? q.w + k : q.w;
            }
            if constexpr (V1) {
                const float4 q = *(const float4 *) (a.v1 + col + e);
                c1[j][e + 0]   = q.x;
                c1[j][e + 1]   = q.y;
                c1[j][e + 2]   = q.z;
                c1[j][e + 3]   = q.w;
            }
        }
    }

    for (uint32_t rbase = blockIdx.x * R; rbase < a.rows; rbase += gridDim.x * R) {
        uint4 ra[R][C], rb[R][C];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = rbase + r;
            if (row < a.rows) {
                const char * ap = a.a + a.ar.off(row);
                const char * bp = LB ? a.b + a.br.off(row) : nullptr;
#pragma unroll
                for (int j = 0; j < C; ++j) {
                    const size_t o = (size_t) ((j * T + tid) * VI) * ES;
                    ra[r][j]       = ld16(ap + o);
                    if constexpr (LB) {
                        rb[r][j] = ld16(bp + o);
                    }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint32_t row = rbase + r;
            if (row >= a.rows) {
                continue;
            }
            char * yp = a.y + a.yr.off(row);
#pragma unroll
            for (int j = 0; j < C; ++j) {
                float fa[VI], fb[VI], fy[VI];
                unpack16<T_>(ra[r][j], fa);
                if constexpr (LB) {
                    unpack16<T_>(rb[r][j], fb);
                }
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    float v = bin_apply<OP, BROW>(fa[e], LB ? fb[e] : 0.0f, V0 ? c0[j][e] : 0.0f,
                                                  V1 ? c1[j][e] : 0.0f);
                    if (a.clamp) {
                        v = clamp_ggml(v, a.lo, a.hi);
                    }
                    fy[e] = v;
                }
                st16(yp + (size_t) ((j * T + tid) * VI) * ES, pack16<T_>(fy));
            }
        }
    }
}

#ifndef MI_BIN_FLAT
#define MI_BIN_FLAT 1  // flat one-shot grid (U vectors per thread) instead of row-stationary
#endif
#ifndef MI_BIN_U
#define MI_BIN_U 1
#endif

// Flat one-shot grid: thread (block b, lane t) handles vectors
// v = b*256*U + k*256 + t of the [rows x nvr] vector grid. Rows are uniformly
// strided (row r at r * nb1 for every operand); the clamp is a template
// parameter, so neither costs instructions when unused. The F32 column
// vectors are read through the caches (a few KB, shared by every row).
template <int T_, int OP, bool BROW, int U, bool CLAMP>
__global__ void __launch_bounds__(256) k_bin_flat(const BinArgs a, uint32_t nvr, FastDiv dnvr, uint32_t total) {
    constexpr int  VI = TT<T_>::VEC;
    constexpr int  ES = TT<T_>::ES;
    constexpr bool V0 = (OP == OP_GATED || OP == OP_MOD || ((OP == OP_ADD || OP == OP_MUL) && !BROW));
    constexpr bool V1 = (OP == OP_MOD);
    constexpr bool LB = BROW || OP == OP_GATED;
    const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
    uint4          ra[U], rb[U];
    uint32_t       row[U], col[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t v = base + k * 256u;
        if (v < total) {
            row[k] = dnvr.div(v);
            col[k] = v - row[k] * nvr;
            ra[k]  = ld16(a.a + (int64_t) row[k] * a.ar.s1 + (size_t) col[k] * 16);
            if constexpr (LB) {
                rb[k] = ld16(a.b + (int64_t) row[k] * a.br.s1 + (size_t) col[k] * 16);
            }
        }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t v = base + k * 256u;
        if (v >= total) {
            continue;
        }
        float fa[VI], fb[VI], fy[VI], c0[VI], c1[VI];
        unpack16<T_>(ra[k], fa);
        if constexpr (LB) {
            unpack16<T_>(rb[k], fb);
        }
        const int c = (int) col[k] * VI;
#pragma unroll
        for (int e = 0; e < VI; e += 4) {
            if constexpr (V0) {
                const float4 q = *(const float4 *) (a.v0 + c + e);
                c0[e + 0]      = OP == OP_MOD ? q.x + 1.0f : q.x;
                c0[e + 1]      = OP == OP_MOD ? q.y + 1.0f : q.y;
                c0[e + 2]      = OP == OP_MOD ? q.z + 1.0f : q.z;
                c0[e + 3]      = OP == OP_MOD ? q.w + 1.0f : q.w;
            }
            if constexpr (V1) {
                const float4 q = *(const float4 *) (a.v1 + c + e);
                c1[e + 0]      = q.x;
                c1[e + 1]      = q.y;
                c1[e + 2]      = q.z;
                c1[e + 3]      = q.w;
            }
        }
#pragma unroll
        for (int e = 0; e < VI; ++e) {
            float v = bin_apply<OP, BROW>(fa[e], LB ? fb[e] : 0.0f, V0 ? c0[e] : 0.0f, V1 ? c1[e] : 0.0f);
            if constexpr (CLAMP) {
                v = clamp_ggml(v, a.lo, a.hi);
            }
            fy[e] = v;
        }
        st16(a.y + (int64_t) row[k] * a.yr.s1 + (size_t) col[k] * VI * ES, pack16<T_>(fy));
    }
}

// Generic path: any types, any strides, ggml_can_repeat broadcast of b.
struct BinGenArgs {
    const char *  a;
    const char *  b;
    char *        y;
    int           ta, tb, ty;
    int64_t       ne[4], anb[4], bne[4], bnb[4], ynb[4];
    const float * v0;
    const float * v1;
    int           op;
    int           clamp;
    float         lo, hi;
};

__device__ __forceinline__ float ld_any(int t, const char * p) {
    switch (t) {
        case MI_TYPE_F32:
            return load_elem<MI_TYPE_F32>(p);
        case MI_TYPE_BF16:
            return load_elem<MI_TYPE_BF16>(p);
        default:
            return load_elem<MI_TYPE_F16>(p);
    }
}

__device__ __forceinline__ void st_any(int t, char * p, float v) {
    switch (t) {
        case MI_TYPE_F32:
            store_elem<MI_TYPE_F32>(p, v);
            break;
        case MI_TYPE_BF16:
            store_elem<MI_TYPE_BF16>(p, v);
            break;
        default:
            store_elem<MI_TYPE_F16>(p, v);
            break;
    }
}

__global__ void __launch_bounds__(256) k_bin_generic(const BinGenArgs g) {
    const uint64_t total = (uint64_t) g.ne[0] * g.ne[1] * g.ne[2] * g.ne[3];
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t) gridDim.x * blockDim.x) {
        uint64_t       q  = i;
        const int64_t  i0 = (int64_t) (q % g.ne[0]);
        q /= g.ne[0];
        const int64_t i1 = (int64_t) (q % g.ne[1]);
        q /= g.ne[1];
        const int64_t i2 = (int64_t) (q % g.ne[2]);
        const int64_t i3 = (int64_t) (q / g.ne[2]);
        const float   av = ld_any(g.ta, g.a + i0 * g.anb[0] + i1 * g.anb[1] + i2 * g.anb[2] + i3 * g.anb[3]);
        float         bv = 0.0f;
        if (g.b) {
            bv = ld_any(g.tb, g.b + (i0 % g.bne[0]) * g.bnb[0] + (i1 % g.bne[1]) * g.bnb[1] +
                                  (i2 % g.bne[2]) * g.bnb[2] + (i3 % g.bne[3]) * g.bnb[3]);
        }
        float v;
        switch (g.op) {
            case OP_ADD:
                v = g.b ? av + bv : av + g.v0[i0];
                break;
            case OP_MUL:
                v = g.b ? av * bv : av * g.v0[i0];
                break;
            case OP_GATED: {
                const float t = bv * g.v0[i0];
                v             = av + t;
                break;
            }
            case OP_MOD: {
                const float sp = g.v0[i0] + 1.0f;
                const float m  = av * sp;
                v              = m + g.v1[i0];
                break;
            }
            default:
                v = av;
                break;
        }
        if (g.clamp) {
            v = clamp_ggml(v, g.lo, g.hi);
        }
        st_any(g.ty, g.y + i0 * g.ynb[0] + i1 * g.ynb[1] + i2 * g.ynb[2] + i3 * g.ynb[3], v);
    }
}

static uint32_t balanced_grid(uint32_t rows, int R, int nw) {
    const uint32_t iters  = (rows + R - 1) / R;
    const uint32_t max_wg = (uint32_t) num_cus() * (uint32_t) (16 / nw > 0 ? 16 / nw : 1);
    const uint32_t per    = (iters + max_wg - 1) / max_wg;
    return (iters + per - 1) / per;
}

template <int T_, int OP, bool BROW>
static int launch_rows_c(const BinArgs & a, int T, int C, hipStream_t s) {
    const int nw = T / 64;
    switch (C) {
        case 1:
            MI_LAUNCH((k_bin_rows<T_, OP, BROW, 1, 4>), dim3(balanced_grid(a.rows, 4, nw)), dim3(T), 0, s, a);
            return MI_OK;
        case 2:
            MI_LAUNCH((k_bin_rows<T_, OP, BROW, 2, 2>), dim3(balanced_grid(a.rows, 2, nw)), dim3(T), 0, s, a);
            return MI_OK;
        case 4:
            MI_LAUNCH((k_bin_rows<T_, OP, BROW, 4, 1>), dim3(balanced_grid(a.rows, 1, nw)), dim3(T), 0, s, a);
            return MI_OK;
        default:
            return MI_ERR_UNSUPPORTED;
    }
}

template <int T_, int OP, bool BROW>
static int launch_flat_op(const BinArgs & a, hipStream_t s) {
    constexpr int  VI    = TT<T_>::VEC;
    const uint32_t nvr   = (uint32_t) (a.n / VI);
    const uint64_t total = (uint64_t) a.rows * nvr;
    const uint32_t grid  = (uint32_t) ((total + 256u * MI_BIN_U - 1) / (256u * MI_BIN_U));
    if constexpr (OP == OP_ADD || OP == OP_NONE) {
        if (a.clamp) {
            MI_LAUNCH((k_bin_flat<T_, OP, BROW, MI_BIN_U, true>), dim3(grid), dim3(256), 0, s, a, nvr,
                               FastDiv(nvr), (uint32_t) total);
            return MI_OK;
        }
    }
    MI_LAUNCH((k_bin_flat<T_, OP, BROW, MI_BIN_U, false>), dim3(grid), dim3(256), 0, s, a, nvr,
                       FastDiv(nvr), (uint32_t) total);
    return MI_OK;
}

template <int T_>
static int launch_flat(int op, bool brow, const BinArgs & a, hipStream_t s) {
    switch (op) {
        case OP_ADD:
            return brow ? launch_flat_op<T_, OP_ADD, true>(a, s) : launch_flat_op<T_, OP_ADD, false>(a, s);
        case OP_MUL:
            return brow ? launch_flat_op<T_, OP_MUL, true>(a, s) : launch_flat_op<T_, OP_MUL, false>(a, s);
        case OP_GATED:
            return launch_flat_op<T_, OP_GATED, true>(a, s);
        case OP_MOD:
            return launch_flat_op<T_, OP_MOD, false>(a, s);
        default:
            return launch_flat_op<T_, OP_NONE, false>(a, s);
    }
}

template <int T_>
static int launch_rows_op(int op, bool brow, const BinArgs & a, int T, int C, hipStream_t s) {
    switch (op) {
        case OP_ADD:
            return brow ? launch_rows_c<T_, OP_ADD, true>(a, T, C, s) : launch_rows_c<T_, OP_ADD, false>(a, T, C, s);
        case OP_MUL:
            return brow ? launch_rows_c<T_, OP_MUL, true>(a, T, C, s) : launch_rows_c<T_, OP_MUL, false>(a, T, C, s);
        case OP_GATED:
            return launch_rows_c<T_, OP_GATED, true>(a, T, C, s);
        case OP_MOD:
            return launch_rows_c<T_, OP_MOD, false>(a, T, C, s);
        default:
            return launch_rows_c<T_, OP_NONE, false>(a, T, C, s);
    }
}

static int launch_generic(int op, const mi_tensor & a, const mi_tensor * b, const float * v0, const float * v1,
                          bool clamp, float lo, float hi, const mi_tensor & y, hipStream_t s) {
    BinGenArgs g;
    g.a  = (const char *) a.data;
    g.b  = b ? (const char *) b->data : nullptr;
    g.y  = (char *) y.data;
    g.ta = a.type;
    g.tb = b ? b->type : MI_TYPE_F32;
    g.ty = y.type;
    for (int d = 0; d < 4; ++d) {
        g.ne[d]  = a.ne[d];
        g.anb[d] = (int64_t) a.nb[d];
        g.ynb[d] = (int64_t) y.nb[d];
        g.bne[d] = b ? b->ne[d] : 1;
        g.bnb[d] = b ? (int64_t) b->nb[d] : 0;
    }
    g.v0    = v0;
    g.v1    = v1;
    g.op    = op;
    g.clamp = clamp;
    g.lo    = lo;
    g.hi    = hi;
    const uint64_t total = (uint64_t) nelements(a);
    if (total == 0) {
        return MI_OK;
    }
    uint64_t       grid = (total + 255) / 256;
    const uint64_t cap  = (uint64_t) num_cus() * 32;
    grid                = grid > cap ? cap : grid;
    MI_LAUNCH(k_bin_generic, dim3((uint32_t) grid), dim3(256), 0, s, g);
    return MI_OK;
}

int launch_binary(int op, const mi_tensor & a, const mi_tensor * b, const float * v0, const float * v1, bool clamp,
                  float lo, float hi, const mi_tensor & y, hipStream_t s) {
    if (nelements(a) == 0) {
        return MI_OK;
    }
    BinArgs k;
    k.a     = (const char *) a.data;
    k.b     = b ? (const char *) b->data : nullptr;
    k.y     = (char *) y.data;
    k.ar    = make_rows3(a);
    k.br    = b ? make_rows3(*b) : make_rows3(a);
    k.yr    = make_rows3(y);
    k.v0    = v0;
    k.v1    = v1;
    k.rows  = (uint32_t) nrows(a);
    k.n     = (int) a.ne[0];
    k.clamp = clamp;
    k.lo    = lo;
    k.hi    = hi;

    bool      fast = a.type == y.type && (!b || b->type == a.type) && is_act(a.type);
    const int VI   = fast ? 16 / type_size(a.type) : 1;
    // flat one-shot path: rows of whole 16-byte vectors, 16-byte aligned
    bool flat = MI_BIN_FLAT && fast && k.n % VI == 0 && aligned(a.data, 16) && aligned(y.data, 16) &&
                (!b || aligned(b->data, 16)) && (!v0 || aligned(v0, 16)) && (!v1 || aligned(v1, 16)) &&
                (uint64_t) k.rows * (k.n / VI) < (1ull << 31);
    for (int d = 1; d < 4 && flat; ++d) {
        flat = a.nb[d] % 16 == 0 && y.nb[d] % 16 == 0 && (!b || b->nb[d] % 16 == 0);
    }
    // rows at r * nb1 in every operand (the flat kernel's addressing)
    flat = flat && k.ar.uni && k.yr.uni && (!b || k.br.uni);
    if (flat) {
        switch (a.type) {
            case MI_TYPE_F32:
                return launch_flat<MI_TYPE_F32>(op, b != nullptr, k, s);
            case MI_TYPE_BF16:
                return launch_flat<MI_TYPE_BF16>(op, b != nullptr, k, s);
            default:
                return launch_flat<MI_TYPE_F16>(op, b != nullptr, k, s);
        }
    }
    int       T = 0, C = 0;
    if (fast && k.n % (64 * VI) == 0) {
        const int kc = k.n / (64 * VI);
        int       nw = 1;
        for (int d = 8; d >= 1; --d) {
            if (kc % d == 0) {
                nw = d;
                break;
            }
        }
        T = nw * 64;
        C = kc / nw;
    }
    fast = fast && (C == 1 || C == 2 || C == 4);
    fast = fast && aligned(a.data, 16) && aligned(y.data, 16) && (!b || aligned(b->data, 16)) &&
           (!v0 || aligned(v0, 16)) && (!v1 || aligned(v1, 16));
    for (int d = 1; d < 4 && fast; ++d) {
        fast = a.nb[d] % 16 == 0 && y.nb[d] % 16 == 0 && (!b || b->nb[d] % 16 == 0);
    }
    if (!fast) {
        return launch_generic(op, a, b, v0, v1, clamp, lo, hi, y, s);
    }
    const bool brow = b != nullptr;
    switch (a.type) {
        case MI_TYPE_F32:
            return launch_rows_op<MI_TYPE_F32>(op, brow, k, T, C, s);
        case MI_TYPE_BF16:
            return launch_rows_op<MI_TYPE_BF16>(op, brow, k, T, C, s);
        default:
            return launch_rows_op<MI_TYPE_F16>(op, brow, k, T, C, s);
    }
}

int launch_binary_bcast(int op, const mi_tensor & a, const mi_tensor & b, bool clamp, float lo, float hi,
                        const mi_tensor & y, hipStream_t s) {
    return launch_generic(op, a, &b, nullptr, nullptr, clamp, lo, hi, y, s);
}

}  // namespace mi
