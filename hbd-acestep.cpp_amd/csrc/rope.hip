// rope.hip -- per-head RMSNorm (QK-norm) fused with NEOX rotary embedding.
//
// ggml node chain reproduced for each head row of D elements (reference:
// qwen3-lm.h:372-379, 660-667; qwen3-enc.h:165-174; dit-graph.h:183-196):
//   n = rms_norm(x, eps) * w                      (optional)
//   ggml_rope_ext mode 2 (NEOX): for pair i < n_dims/2
//     theta_0 = (float)pos, theta_{i+1} = theta_i * theta_scale   (fp32 chain)
//     c = cosf(freq_scale*theta_i)*attn_factor, s = sinf(...)*attn_factor
//     (cos/sin evaluated in double, rounded once to fp32)
//     y_i = n_i*c - n_{i+h}*s ;  y_{i+h} = n_i*s + n_{i+h}*c     (h = n_dims/2)
// theta_scale = powf(freq_base, -2/n_dims) is computed on the host, with the
// host libm, as ggml-cpu does.
//
// Fast path (n_dims == ne0 == D in {64, 128, 256}): a lane holds 16 bytes of
// the first half of a head row and the matching 16 bytes of the second
// half, so both members of every rotated pair are in the same lane (no
// cross-lane exchange for the rotation). A head row is spread over
// L = D/2/VEC lanes and reduced with DPP. Each workgroup covers TPB tokens;
// their cos/sin tables (one (pos, pair) per thread) are built once in LDS and
// shared by all Q and K heads of those tokens. Inputs may be strided views of
// the fused QKV projection output, so no separate contiguous copy is needed.
#include "launch.h"

namespace mi {

template <int TI, int TO, int D, bool NORM, bool ROPE>
__global__ void __launch_bounds__(256) k_heads(const HeadArgs a) {
    constexpr int VI   = TT<TI>::VEC;
    constexpr int EI   = TT<TI>::ES;
    constexpr int EO   = TT<TO>::ES;
    constexpr int HALF = D / 2;
    constexpr int L    = HALF / VI;   // lanes per head row
    constexpr int TPB  = 256 / HALF;  // tokens per workgroup
    constexpr int G    = 256 / L;     // head rows in flight per workgroup

    __shared__ f32x2 cs[ROPE ? TPB : 1][ROPE ? HALF : 1];

    const int      tid  = threadIdx.x;
    const uint32_t tok0 = blockIdx.x * TPB;

    if constexpr (ROPE) {
        const int      tt = tid / HALF;
        const int      i  = tid % HALF;
        const uint32_t t  = tok0 + tt;
        float          c = 1.0f, sn = 0.0f;
        if (t < a.ntok) {
            const uint32_t i3    = a.dne2.div(t);
            const uint32_t i2    = t - i3 * a.ne2;
            float          theta = (float) a.pos[i2];
            // theta_i after i sequential fp32 multiplies (the ggml cache chain)
#pragma unroll 8
            for (int k = 0; k < HALF - 1; ++k) {
                const float nt = theta * a.theta_scale;
                theta          = k < i ? nt : theta;
            }
            const float th = a.freq_scale * theta;
            float       sv, cv;
            sincos_f32(th, &sv, &cv);
            c  = cv * a.mscale;
            sn = sv * a.mscale;
        }
        cs[tt][i] = f32x2{ c, sn };
        __syncthreads();
    }

    const int g = tid / L;
    const int j = tid % L;

    for (int sgi = 0; sgi < a.nseg; ++sgi) {
        const HeadSeg & S = a.seg[sgi];
        float           w0[VI], w1[VI];
        if constexpr (NORM) {
#pragma unroll
            for (int e = 0; e < VI; ++e) {
                w0[e] = S.w ? S.w[j * VI + e] : 1.0f;
                w1[e] = S.w ? S.w[HALF + j * VI + e] : 1.0f;
            }
        }
        const bool     has_w = S.w != nullptr;
        const uint32_t nrows = TPB * S.heads;
        for (uint32_t r = g; r < nrows; r += G) {
            const uint32_t tt = S.hdiv.div(r);
            const uint32_t h  = r - tt * S.heads;
            const uint32_t t  = tok0 + tt;
            if (t >= a.ntok) {
                continue;
            }
            const uint32_t i3 = a.dne2.div(t);
            const uint32_t i2 = t - i3 * a.ne2;
            const char *   xp = S.x + (int64_t) i3 * S.xs3 + (int64_t) i2 * S.xs2 + (int64_t) h * S.xs1;
            char *         yp = S.y + (int64_t) i3 * S.ys3 + (int64_t) i2 * S.ys2 + (int64_t) h * S.ys1;
            const uint4    v0 = ld16(xp + (size_t) (j * VI) * EI);
            const uint4    v1 = ld16(xp + (size_t) (HALF + j * VI) * EI);
            float          x0[VI], x1[VI];
            unpack16<TI>(v0, x0);
            unpack16<TI>(v1, x1);
            if constexpr (NORM) {
                double s = 0.0;
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    s += (double) (x0[e] * x0[e]);
                }
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    s += (double) (x1[e] * x1[e]);
                }
                s                 = group_sum<L>(s);
                const float scale = rms_scale(s, D, a.eps);
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    x0[e] = x0[e] * scale;
                    x1[e] = x1[e] * scale;
                }
                if (has_w) {
#pragma unroll
                    for (int e = 0; e < VI; ++e) {
                        x0[e] = x0[e] * w0[e];
                        x1[e] = x1[e] * w1[e];
                    }
                }
            }
            if constexpr (ROPE) {
#pragma unroll
                for (int e = 0; e < VI; ++e) {
                    const f32x2 q  = cs[tt][j * VI + e];
                    const float a0 = x0[e] * q.x;
                    const float b0 = x1[e] * q.y;
                    const float a1 = x0[e] * q.y;
                    const float b1 = x1[e] * q.x;
                    x0[e]          = a0 - b0;
                    x1[e]          = a1 + b1;
                }
            }
            store_vec<TO, VI>(yp + (size_t) (j * VI) * EO, x0);
            store_vec<TO, VI>(yp + (size_t) (HALF + j * VI) * EO, x1);
        }
    }
}

// Generic path: any ne0 / n_dims (even, <= ne0), element-aligned rows.
// One wave per head row; each lane derives the theta chain of its own pairs.
template <int TI, int TO>
__global__ void __launch_bounds__(256) k_heads_generic(const HeadArgs a) {
    constexpr int EI   = TT<TI>::ES;
    constexpr int EO   = TT<TO>::ES;
    const int     lane = threadIdx.x & 63;
    const int     wpb  = blockDim.x >> 6;
    const int     half = a.n_dims / 2;
    for (int sgi = 0; sgi < a.nseg; ++sgi) {
        const HeadSeg & S     = a.seg[sgi];
        const uint64_t  nrows = (uint64_t) a.ntok * S.heads;
        for (uint64_t r = (uint64_t) blockIdx.x * wpb + (threadIdx.x >> 6); r < nrows; r += (uint64_t) gridDim.x * wpb) {
            const uint32_t t  = (uint32_t) (r / S.heads);
            const uint32_t h  = (uint32_t) (r - (uint64_t) t * S.heads);
            const uint32_t i3 = a.dne2.div(t);
            const uint32_t i2 = t - i3 * a.ne2;
            const char *   xp = S.x + (int64_t) i3 * S.xs3 + (int64_t) i2 * S.xs2 + (int64_t) h * S.xs1;
            char *         yp = S.y + (int64_t) i3 * S.ys3 + (int64_t) i2 * S.ys2 + (int64_t) h * S.ys1;
            float          scale = 1.0f;
            if (a.norm) {
                double s = 0.0;
                for (int i = lane; i < a.ne0; i += 64) {
                    const float f = load_elem<TI>(xp + (size_t) i * EI);
                    s += (double) (f * f);
                }
                s     = group_sum<64>(s);
                scale = rms_scale(s, a.ne0, a.eps);
            }
            auto nval = [&](int i) {
                float v = load_elem<TI>(xp + (size_t) i * EI);
                if (a.norm) {
                    v = v * scale;
                    if (S.w) {
                        v = v * S.w[i];
                    }
                }
                return v;
            };
            if (a.pos) {
                const float p = (float) a.pos[i2];
                for (int ic = lane; ic < half; ic += 64) {
                    float theta = p;
                    for (int k = 0; k < ic; ++k) {
                        theta = theta * a.theta_scale;
                    }
                    const float th = a.freq_scale * theta;
                    float       sv, cv;
                    sincos_f32(th, &sv, &cv);
                    const float c  = cv * a.mscale;
                    const float sn = sv * a.mscale;
                    const float x0 = nval(ic);
                    const float x1 = nval(ic + half);
                    const float a0 = x0 * c;
                    const float b0 = x1 * sn;
                    const float a1 = x0 * sn;
                    const float b1 = x1 * c;
                    store_elem<TO>(yp + (size_t) ic * EO, a0 - b0);
                    store_elem<TO>(yp + (size_t) (ic + half) * EO, a1 + b1);
                }
                for (int i = a.n_dims + lane; i < a.ne0; i += 64) {
                    store_elem<TO>(yp + (size_t) i * EO, nval(i));
                }
            } else {
                for (int i = lane; i < a.ne0; i += 64) {
                    store_elem<TO>(yp + (size_t) i * EO, nval(i));
                }
            }
        }
    }
}

template <int TI, int TO, int D>
static void launch_fast(const HeadArgs & a, hipStream_t s) {
    constexpr int  TPB  = 256 / (D / 2);
    const uint32_t grid = (a.ntok + TPB - 1) / TPB;
    const bool     rope = a.pos != nullptr;
    if (a.norm && rope) {
        hipLaunchKernelGGL((k_heads<TI, TO, D, true, true>), dim3(grid), dim3(256), 0, s, a);
    } else if (a.norm) {
        hipLaunchKernelGGL((k_heads<TI, TO, D, true, false>), dim3(grid), dim3(256), 0, s, a);
    } else {
        hipLaunchKernelGGL((k_heads<TI, TO, D, false, true>), dim3(grid), dim3(256), 0, s, a);
    }
}

template <int TI, int TO>
static int launch_t(HeadArgs & a, bool fast, hipStream_t s) {
    if (fast) {
        for (int i = 0; i < a.nseg; ++i) {
            a.seg[i].hdiv = FastDiv(a.seg[i].heads);
        }
        switch (a.ne0) {
            case 64:
                launch_fast<TI, TO, 64>(a, s);
                return MI_OK;
            case 128:
                launch_fast<TI, TO, 128>(a, s);
                return MI_OK;
            case 256:
                launch_fast<TI, TO, 256>(a, s);
                return MI_OK;
            default:
                break;
        }
    }
    uint64_t rows = 0;
    for (int i = 0; i < a.nseg; ++i) {
        rows = rows > (uint64_t) a.ntok * a.seg[i].heads ? rows : (uint64_t) a.ntok * a.seg[i].heads;
    }
    uint64_t grid = (rows + 3) / 4;
    const uint64_t cap = (uint64_t) num_cus() * 16;
    grid = grid > cap ? cap : (grid ? grid : 1);
    hipLaunchKernelGGL((k_heads_generic<TI, TO>), dim3((uint32_t) grid), dim3(256), 0, s, a);
    return MI_OK;
}

int launch_heads(HeadArgs & a, int tin, int tout, hipStream_t s) {
    if (a.ntok == 0) {
        return MI_OK;
    }
    a.dne2 = FastDiv(a.ne2);
    // fast path preconditions: full-width rotation (or none), D in {64,128,256},
    // 16-byte aligned rows, same in/out type
    bool fast = (a.pos == nullptr || a.n_dims == a.ne0) && (a.ne0 == 64 || a.ne0 == 128 || a.ne0 == 256) &&
                tin == tout && (a.norm || a.pos);
    for (int i = 0; i < a.nseg && fast; ++i) {
        const HeadSeg & S = a.seg[i];
        fast = aligned(S.x, 16) && aligned(S.y, 16) && S.xs1 % 16 == 0 && S.xs2 % 16 == 0 && S.xs3 % 16 == 0 &&
               S.ys1 % 16 == 0 && S.ys2 % 16 == 0 && S.ys3 % 16 == 0 && (!S.w || aligned(S.w, 16));
    }
    switch (tin) {
        case MI_TYPE_F32:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_F32, MI_TYPE_F32>(a, fast, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_F32, MI_TYPE_BF16>(a, false, s);
                default:
                    return launch_t<MI_TYPE_F32, MI_TYPE_F16>(a, false, s);
            }
        case MI_TYPE_BF16:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_F32>(a, false, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_BF16>(a, fast, s);
                default:
                    return launch_t<MI_TYPE_BF16, MI_TYPE_F16>(a, false, s);
            }
        default:
            switch (tout) {
                case MI_TYPE_F32:
                    return launch_t<MI_TYPE_F16, MI_TYPE_F32>(a, false, s);
                case MI_TYPE_BF16:
                    return launch_t<MI_TYPE_F16, MI_TYPE_BF16>(a, false, s);
                default:
                    return launch_t<MI_TYPE_F16, MI_TYPE_F16>(a, fast, s);
            }
    }
}

}  // namespace mi
