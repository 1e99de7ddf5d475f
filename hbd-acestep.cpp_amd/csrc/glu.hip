// glu.hip -- SwiGLU: y = silu(g) * u, silu(x) = x / (1 + e^-x).
//
// Replaces ggml_swiglu (fused [2I] gate|up rows, gate = first half) and
// ggml_swiglu_split (reference: qwen3-enc.h:209-224, dit-graph.h:250-269).
//
// The exponential is v_exp_f32 (2^t) on t = -x*log2(e), with the rounding
// error of that product recovered by an fma and folded back in first order,
// so e^-x is good to ~1 ulp over the whole finite range; the quotient is
// x * v_rcp_f32(1 + e^-x). Relative error vs x/(1.0f + expf(-x)) stays a few
// ulp (<1e-6). For x < -88.7, e^-x overflows to +inf exactly as expf does in
// ggml, and the result is -0 like ggml's x/inf.
//
// Memory layout: rows are uniformly strided (ggml requires contiguous rows
// here); each thread moves U 16-byte vectors of g and u with all loads issued
// before any math.
#include "launch.h"

namespace mi {


struct GluArgs {
    const char * g;
    const char * u;
    char *       y;
    int64_t      gs, us, ys;  // row strides, bytes
    uint32_t     nvr;         // 16-byte input vectors per row
    FastDiv      dnvr;
    uint32_t     total;       // rows * nvr
};

template <int TI, int TO, int U>
__global__ void __launch_bounds__(256) k_swiglu(const GluArgs a) {
    constexpr int  VI   = TT<TI>::VEC;
    constexpr int  EO   = TT<TO>::ES;
    const uint32_t base = blockIdx.x * (256u * U) + threadIdx.x;
    uint4          gv[U], uv[U];
    uint32_t       row[U], col[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t v = base + k * 256u;
        if (v < a.total) {
            row[k] = a.dnvr.div(v);
            col[k] = v - row[k] * a.nvr;
            gv[k]  = ld16(a.g + (int64_t) row[k] * a.gs + (size_t) col[k] * 16);
            uv[k]  = ld16(a.u + (int64_t) row[k] * a.us + (size_t) col[k] * 16);
        }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t v = base + k * 256u;
        if (v < a.total) {
            float g[VI], u[VI], y[VI];
            unpack16<TI>(gv[k], g);
            unpack16<TI>(uv[k], u);
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                y[e] = silu_f(g[e]) * u[e];
            }
            store_vec<TO, VI>(a.y + (int64_t) row[k] * a.ys + (size_t) col[k] * VI * EO, y);
        }
    }
}

template <int TI, int TO>
__global__ void __launch_bounds__(256) k_swiglu_generic(const char * g, const char * u, int64_t gs, int64_t us,
                                                        char * y, int64_t ys, int64_t rows, int64_t n) {
    constexpr int  EI    = TT<TI>::ES;
    constexpr int  EO    = TT<TO>::ES;
    const uint64_t total = (uint64_t) rows * (uint64_t) n;
    for (uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (uint64_t) gridDim.x * blockDim.x) {
        const uint64_t r  = i / (uint64_t) n;
        const uint64_t c  = i - r * (uint64_t) n;
        const float    gv = load_elem<TI>(g + (int64_t) r * gs + c * EI);
        const float    uv = load_elem<TI>(u + (int64_t) r * us + c * EI);
        store_elem<TO>(y + (int64_t) r * ys + c * EO, silu_f(gv) * uv);
    }
}

#ifndef MI_GLU_U
#define MI_GLU_U 2  // 16-byte vectors of g and u per thread
#endif

template <int TI, int TO>
static int launch_t(const GluArgs & a, bool fast, int64_t rows, int64_t n, hipStream_t s) {
    if (fast) {
        constexpr int  U    = MI_GLU_U;
        const uint32_t grid = (a.total + 256u * U - 1) / (256u * U);
        MI_LAUNCH((k_swiglu<TI, TO, U>), dim3(grid), dim3(256), 0, s, a);
        return MI_OK;
    }
    uint64_t       grid = ((uint64_t) rows * n + 255) / 256;
    const uint64_t cap  = (uint64_t) num_cus() * 32;
    grid                = grid > cap ? cap : (grid ? grid : 1);
    MI_LAUNCH((k_swiglu_generic<TI, TO>), dim3((uint32_t) grid), dim3(256), 0, s, a.g, a.u, a.gs, a.us,
                       a.y, a.ys, rows, n);
    return MI_OK;
}

int launch_swiglu(const char * g, const char * u, int64_t gs, int64_t us, int tin, char * y, int64_t ys, int tout,
                  int64_t rows, int64_t n, bool vec_ok, hipStream_t s) {
    if (rows == 0 || n == 0) {
        return MI_OK;
    }
    const int VI = 16 / type_size(tin);
    GluArgs   a;
    a.g  = g;
    a.u  = u;
    a.y  = y;
    a.gs = gs;
    a.us = us;
    a.ys = ys;
    bool fast = vec_ok && tin == tout && n % VI == 0 && aligned(g, 16) && aligned(u, 16) && aligned(y, 16) &&
                gs % 16 == 0 && us % 16 == 0 && ys % 16 == 0 && (uint64_t) rows * (n / VI) < (1ull << 31);
    if (fast) {
        a.nvr   = (uint32_t) (n / VI);
        a.dnvr  = FastDiv(a.nvr);
        a.total = (uint32_t) (rows * a.nvr);
    }
    switch (tin) {
        case MI_TYPE_F32:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_F32, MI_TYPE_F32>(a, fast, rows, n, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_F32, MI_TYPE_BF16>(a, false, rows, n, s);
                default:
                    return launch_t<MI_TYPE_F32, MI_TYPE_F16>(a, false, rows, n, s);
            }
        case MI_TYPE_BF16:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_F32>(a, false, rows, n, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_BF16>(a, fast, rows, n, s);
                default:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_F16>(a, false, rows, n, s);
            }
        default:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_F16, MI_TYPE_F32>(a, false, rows, n, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_F16, MI_TYPE_BF16>(a, false, rows, n, s);
                default:
                    return launch_t<MI_TYPE_F16, MI_TYPE_F16>(a, fast, rows, n, s);
            }
    }
}

}  // namespace mi
