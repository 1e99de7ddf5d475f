// tsembd.hip -- ggml_timestep_embedding (reference: dit-graph.h:81-117, the
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

int launch_timestep_embedding(const float * t, int64_t n, int64_t ts, int dim, int max_period, char * y,
                              int64_t ys, hipStream_t s) {
    const int64_t total = n * (int64_t) (dim / 2 + 1);
    if (total == 0) {
        return MI_OK;
    }
    int64_t grid = (total + 255) / 256;
    grid         = grid > 1024 ? 1024 : grid;
    hipLaunchKernelGGL(k_tsembd, dim3((uint32_t) grid), dim3(256), 0, s, t, n, ts, dim, max_period, y, ys);
    return MI_OK;
}

}  // namespace mi
