// tsembd.hip -- ggml_scale, which scales the timestep by 1000 in front of the
// embedding (dit-graph.h:87), and ggml_timestep_embedding (dit-graph.h:81-117, the
// DiT's sinusoidal timestep embedding, dim 256, max_period 10000):
//   half = dim/2; freq_j = expf(-logf(max_period) * j / half)
//   y[j] = cosf(t * freq_j); y[j + half] = sinf(t * freq_j); odd dim -> y[2*half] = 0
// Tiny (dim floats per step); one thread per (t, j). The fp32 argument
// chain is rounded exactly as written above; exp/log/cos/sin are evaluated
// in double and rounded once.
#include "launch.h"

namespace mi {

__global__ void __launch_bounds__(256) k_tsembd(const float * t, int64_t n, int64_t ts, int dim, int max_period,
                                                char * y, int64_t ys) {
    const int half = dim / 2;
    const int64_t total = n * (int64_t) (half + 1);
    for (int64_t g = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; g < total; g += (int64_t) gridDim.x * blockDim.x) {
        const int64_t i  = g / (half + 1);
        const int     j  = (int) (g - i * (half + 1));
        float *       yr = (float *) (y + i * ys);
        if (j == half) {
            if (dim % 2 != 0) {
                yr[2 * half] = 0.0f;
            }
            continue;
        }
        const float timestep = t[i * ts];
        const float lp       = -log_f32((float) max_period);
        const float ex       = lp * (float) j / (float) half;
        const float freq     = exp_f32(ex);
        const float arg      = timestep * freq;
        float       sv, cv;
        sincos_f32(arg, &sv, &cv);
        yr[j]        = cv;
        yr[j + half] = sv;
    }
}

// y = x * s per element (rows addressed through Rows3, elements contiguous);
// tiny in its one use (a [1] timestep), so a plain grid-stride loop
template <int TI, int TO>
__global__ void __launch_bounds__(256) k_scale(const char * x, Rows3 xr, char * y, Rows3 yr, uint32_t rows,
                                               uint32_t n, float sc) {
    const uint64_t total = (uint64_t) rows * n;
    for (uint64_t g = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; g < total;
         g += (uint64_t) gridDim.x * blockDim.x) {
        const uint64_t row = g / n;
        const uint32_t i   = (uint32_t) (g - row * n);
        const float    v   = load_elem<TI>(x + xr.off((uint32_t) row) + (size_t) i * TT<TI>::ES) * sc;
        store_elem<TO>(y + yr.off((uint32_t) row) + (size_t) i * TT<TO>::ES, v);
    }
}

template <int TI>
static void scale_out(const mi_tensor & x, float sc, const mi_tensor & y, uint32_t grid, hipStream_t s) {
    const Rows3    xr = make_rows3(x), yr = make_rows3(y);
    const uint32_t rows = (uint32_t) nrows(x), n = (uint32_t) x.ne[0];
    switch (y.type) {
        case MI_TYPE_F32:
            MI_LAUNCH((k_scale<TI, MI_TYPE_F32>), dim3(grid), dim3(256), 0, s, (const char *) x.data, xr,
                               (char *) y.data, yr, rows, n, sc);
            break;
        case MI_TYPE_BF16:
            MI_LAUNCH((k_scale<TI, MI_TYPE_BF16>), dim3(grid), dim3(256), 0, s, (const char *) x.data, xr,
                               (char *) y.data, yr, rows, n, sc);
            break;
        default:
            MI_LAUNCH((k_scale<TI, MI_TYPE_F16>), dim3(grid), dim3(256), 0, s, (const char *) x.data, xr,
                               (char *) y.data, yr, rows, n, sc);
            break;
    }
}

int launch_scale(const mi_tensor & x, float sc, const mi_tensor & y, hipStream_t s) {
    const uint64_t total = (uint64_t) nrows(x) * (uint64_t) x.ne[0];
    if (total == 0) {
        return MI_OK;
    }
    uint64_t grid = (total + 255) / 256;
    grid          = grid > 4096 ? 4096 : grid;
    switch (x.type) {
        case MI_TYPE_F32:
            scale_out<MI_TYPE_F32>(x, sc, y, (uint32_t) grid, s);
            break;
        case MI_TYPE_BF16:
            scale_out<MI_TYPE_BF16>(x, sc, y, (uint32_t) grid, s);
            break;
        default:
            scale_out<MI_TYPE_F16>(x, sc, y, (uint32_t) grid, s);
            break;
    }
    return MI_OK;
}

int launch_timestep_embedding(const float * t, int64_t n, int64_t ts, int dim, int max_period, char * y,
                              int64_t ys, hipStream_t s) {
    const int64_t total = n * (int64_t) (dim / 2 + 1);
    if (total == 0) {
        return MI_OK;
    }
    int64_t grid = (total + 255) / 256;
    grid         = grid > 1024 ? 1024 : grid;
    MI_LAUNCH(k_tsembd, dim3((uint32_t) grid), dim3(256), 0, s, t, n, ts, dim, max_period, y, ys);
    return MI_OK;
}

}  // namespace mi
