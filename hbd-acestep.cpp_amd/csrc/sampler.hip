// The DiT sampler's per-step math on the device, so the flow-matching loop
// keeps its latents resident (reference: dit_ggml_generate, dit-sampler.h:408-640,
// which reads the velocity back, applies APG and the solver on the host and
// uploads the next input every step).
//
// APG (apg_forward, dit-sampler.h:66-118; momentum buffer 19-35, projection
// 37-64): per sample, in double,
//   diff = cond - uncond;  ra = first ? diff : diff + momentum * ra
//   per channel c over T:  s = min(1, threshold / |ra_c|) (1 if |ra_c| <= 1e-60)
//                          inv = 1 / |cond_c| (0 if |cond_c|^2 <= 1e-60)
//                          dot = sum_t (s ra) (cond inv)
//   out = (float) (cond + (scale - 1) (s ra - dot cond inv))
// One workgroup per sample: lanes own channels, waves split the frames; the
// three per-channel sums (|ra|^2, |cond|^2, ra . cond) reduce in LDS, then a
// second pass writes the result. Layout [N][T][Oc] (ggml [Oc, T, N]).
//
// Solvers (solvers/solver-euler.h, solver-dpm.h) and the final step
// (dit-sampler.h:601-605), in fp32 with the reference's operation order:
//   euler:  xt -= vt * (t_curr - t_next)
//   dpm3m:  v = (23/12) vt - (16/12) prev + (5/12) prev2  (AB3; AB2 = 1.5 vt - 0.5 prev;
//           Euler first), xt -= v * dt, then prev2 <- prev, prev <- vt
//   final:  out = xt - vt * t
#include "common.h"
#include "launch.h"

namespace mi {

__global__ void __launch_bounds__(1024) k_apg(const ApgArgs a) {
    extern __shared__ double red[];  // [3][nph][oc], then [3][oc]
    const uint32_t b   = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t oc = a.oc, nph = blockDim.x / a.oc;
    const uint32_t c = tid % oc, ph = tid / oc;  // blockDim is nph * oc: every thread has a (channel, phase)
    const float * cond = a.cond + (size_t) b * a.t * oc;
    const float * unc  = a.uncond + (size_t) b * a.t * oc;
    double *      ra   = a.ra + (size_t) b * a.t * oc;
    float *       out  = a.out + (size_t) b * a.t * oc;
    double        s_rr = 0.0, s_cc = 0.0, s_rc = 0.0;
    for (uint32_t t = ph; t < a.t; t += nph) {
        const size_t i  = (size_t) t * oc + c;
        const double cv = (double) cond[i];
        const double d  = cv - (double) unc[i];
        const double r  = a.first ? d : d + a.momentum * ra[i];
        ra[i]           = r;
        s_rr += r * r;
        s_cc += cv * cv;
        s_rc += r * cv;
    }
    red[(0 * nph + ph) * oc + c] = s_rr;
    red[(1 * nph + ph) * oc + c] = s_cc;
    red[(2 * nph + ph) * oc + c] = s_rc;
    __syncthreads();
    double * fin = red + 3 * nph * oc;  // per channel: s, inv, dot
    if (ph == 0) {
        double rr = 0.0, cc = 0.0, rc = 0.0;
        for (uint32_t p = 0; p < nph; ++p) {
            rr += red[(0 * nph + p) * oc + c];
            cc += red[(1 * nph + p) * oc + c];
            rc += red[(2 * nph + p) * oc + c];
        }
        const double norm = sqrt(rr > 0.0 ? rr : 0.0);
        double       s    = 1.0;
        if (a.threshold > 0.0f && norm > 1e-60) {
            s = fmin(1.0, (double) a.threshold / norm);
        }
        const double inv = cc > 1e-60 ? 1.0 / sqrt(cc) : 0.0;
        fin[c]           = s;
        fin[oc + c]      = inv;
        fin[2 * oc + c]  = s * inv * rc;
    }
    __syncthreads();
    const double s = fin[c], inv = fin[oc + c], dot = fin[2 * oc + c];
    const double w = (double) a.scale - 1.0;
    for (uint32_t t = ph; t < a.t; t += nph) {
        const size_t i    = (size_t) t * oc + c;
        const double cv   = (double) cond[i];
        const double orth = s * ra[i] - dot * (cv * inv);
        out[i]            = (float) (cv + w * orth);
    }
}

// solver 0 euler, 1 dpm3m (hist = stored velocities: 0, 1 or 2), 2 final x0,
// 3 sde (x0 = xt - vt t_curr; xt = t_next noise + (1 - t_next) x0)
__global__ void __launch_bounds__(256) k_flow_step(const FlowArgs a) {
    const uint64_t i = (uint64_t) blockIdx.x * 256u + threadIdx.x;
    if (i >= a.n) {
        return;
    }
    const float v = a.vt[i];
    if (a.solver == 2) {
        a.out[i] = a.xt[i] - v * a.t_curr;
        return;
    }
    if (a.solver == 3) {
        const float x0 = a.xt[i] - v * a.t_curr;
        a.xt[i]        = a.t_next * a.noise[i] + (1.0f - a.t_next) * x0;
        return;
    }
    const float dt = a.t_curr - a.t_next;
    float       ve = v;
    if (a.solver == 1) {
        if (a.hist >= 2) {
            const float c0 = 23.0f / 12.0f, c1 = 16.0f / 12.0f, c2 = 5.0f / 12.0f;
            ve = c0 * v - c1 * a.prev[i] + c2 * a.prev2[i];
        } else if (a.hist == 1) {
            ve = 1.5f * v - 0.5f * a.prev[i];
        }
        if (a.hist >= 1) {
            a.prev2[i] = a.prev[i];
        }
        a.prev[i] = v;
    }
    a.xt[i] -= ve * dt;
}

// ---- STORK4 (solvers/solver-stork.h) ----------------------------------------
// Velocity derivatives from the two latest stored velocities (forward
// difference and the three-point formula, solver-stork.h:69-126), recomputed
// bit-identically wherever they are needed instead of being stored.
__device__ __forceinline__ void stork_derivs(const StorkArgs & a, uint64_t i, float v, float & dv, float & d2v) {
    dv = d2v = 0.0f;
    if (a.max_order >= 1) {
        const float p1 = a.prev[i];
        dv             = (p1 - v) / a.h1;
        if (a.max_order >= 2) {
            const double h1 = (double) a.h1, h2 = (double) a.h2;
            d2v = (float) (a.c2 * ((double) a.prev2[i] * h1 - (double) p1 * (h1 + h2) + (double) v * h2));
        }
    }
}

// _stork_taylor_approx (solver-stork.h:45-64): v(t + diff) from v, dv, d2v
__device__ __forceinline__ float stork_vel(int order, float diff, float v, float dv, float d2v) {
    if (order >= 2) {
        const float h = 0.5f * diff * diff;
        return v + diff * dv + h * d2v;
    }
    if (order == 1) {
        return v + diff * dv;
    }
    return v;
}

// Sum of a thread's value over a 256-thread block, in a fixed order; every
// thread receives the total.
__device__ __forceinline__ double block_sum256(double v, double * lds) {
    v = group_sum<64>(v);
    const uint32_t w = threadIdx.x / WAVE;
    __syncthreads();
    if (threadIdx.x % WAVE == 0) {
        lds[w] = v;
    }
    __syncthreads();
    return (lds[0] + lds[1]) + (lds[2] + lds[3]);
}

// Statistics pass: per-block sums of vt^2, dv^2, d2v^2 in double; block 0 also
// clears the attempt flags.
__global__ void __launch_bounds__(256) k_stork_stats(const StorkArgs a) {
    __shared__ double lds[4];
    double            s0 = 0.0, s1 = 0.0, s2 = 0.0;
    const uint64_t    stride = (uint64_t) gridDim.x * 256u;
    for (uint64_t i = (uint64_t) blockIdx.x * 256u + threadIdx.x; i < a.n; i += stride) {
        const float v = a.vt[i];
        float       dv, d2v;
        stork_derivs(a, i, v, dv, d2v);
        s0 += (double) v * (double) v;
        s1 += (double) dv * (double) dv;
        s2 += (double) d2v * (double) d2v;
    }
    s0 = block_sum256(s0, lds);
    s1 = block_sum256(s1, lds);
    s2 = block_sum256(s2, lds);
    if (threadIdx.x == 0) {
        a.part[blockIdx.x * 3 + 0] = s0;
        a.part[blockIdx.x * 3 + 1] = s1;
        a.part[blockIdx.x * 3 + 2] = s2;
    }
    if (blockIdx.x == 0 && threadIdx.x < 4 + STORK_MAX_ATTEMPTS && threadIdx.x >= 1) {
        a.status[threadIdx.x] = 0u;
    }
}

// The derivative order the guards allow (solver-stork.h:84-88, 113-116), from
// the statistics pass's partial sums reduced in a fixed order.
__device__ int stork_order(const StorkArgs & a, uint32_t nblk, double * lds) {
    if (a.max_order == 0) {
        return 0;
    }
    const uint32_t t  = threadIdx.x;
    const double   s0 = block_sum256(t < nblk ? a.part[t * 3 + 0] : 0.0, lds);
    const double   s1 = block_sum256(t < nblk ? a.part[t * 3 + 1] : 0.0, lds);
    const double   s2 = block_sum256(t < nblk ? a.part[t * 3 + 2] : 0.0, lds);
    const double   n  = (double) a.n;
    const double   vr = sqrt(s0 / n), dr = sqrt(s1 / n), d2r = sqrt(s2 / n);
    if (vr > 0.0 && dr * fabs((double) a.h1) > 5.0 * vr) {
        return 0;
    }
    if (a.max_order == 1) {
        return 1;
    }
    if (vr > 0.0 && d2r * (double) a.h1 * (double) a.h1 > 5.0 * vr) {
        return 1;
    }
    return 2;
}

// One sub-stepping attempt (_rock4_substep, solver-stork.h:163-267): the
// Chebyshev recurrence over the plan's degree, then the finishing blend, per
// element in registers. Exits at once when an earlier attempt of this step was
// finite everywhere; flags its own attempt when any result is not finite.
__global__ void __launch_bounds__(256) k_stork_attempt(const StorkArgs a, const StorkPlan p, uint32_t nblk) {
    __shared__ double lds[4];
    for (int q = 0; q < p.attempt; ++q) {
        if (a.status[4 + q] == 0u) {
            return;  // block-uniform
        }
    }
    const int order = stork_order(a, nblk, lds);
    if (p.attempt == 0 && blockIdx.x == 0 && threadIdx.x == 0) {
        a.status[1] = (uint32_t) order;
    }
    const uint64_t stride = (uint64_t) gridDim.x * 256u;
    bool           bad    = false;
    for (uint64_t i = (uint64_t) blockIdx.x * 256u + threadIdx.x; i < a.n; i += stride) {
        const float x = a.xt[i], v = a.vt[i];
        float       dv, d2v;
        stork_derivs(a, i, v, dv, d2v);
        float y2 = x, y1 = x + p.t1_first * v;
        for (int j = 0; j < p.mdeg - 1; ++j) {
            const float vel = stork_vel(order, p.sub[j][3], v, dv, d2v);
            const float yj  = p.sub[j][0] * vel + p.sub[j][1] * y1 + p.sub[j][2] * y2;
            y2              = y1;
            y1              = yj;
        }
        const float f1  = stork_vel(order, p.fin_diff[0], v, dv, d2v);
        const float f2  = stork_vel(order, p.fin_diff[1], v, dv, d2v);
        const float f3  = stork_vel(order, p.fin_diff[2], v, dv, d2v);
        const float f4  = stork_vel(order, p.fin_diff[3], v, dv, d2v);
        const float out = y1 + p.fpb[0] * f1 + p.fpb[1] * f2 + p.fpb[2] * f3 + p.fpb[3] * f4;
        a.xnext[i]      = out;
        bad |= !isfinite(out);
    }
    if (__any(bad) && threadIdx.x % WAVE == 0) {
        atomicOr(&a.status[4 + p.attempt], 1u);
    }
}

// Commit: the first finite attempt's result, or Euler when every attempt failed
// (solver-stork.h:307-318) or at the bootstrap step (289-296); then the history
// rotation prev2 <- prev, prev <- vt (_stork_update_history).
__global__ void __launch_bounds__(256) k_stork_commit(const StorkArgs a) {
    int acc = -1;
    if (a.hist > 0) {
        for (int q = 0; q < a.n_attempts; ++q) {
            if (a.status[4 + q] == 0u) {
                acc = q;
                break;
            }
        }
    }
    const uint64_t stride = (uint64_t) gridDim.x * 256u;
    for (uint64_t i = (uint64_t) blockIdx.x * 256u + threadIdx.x; i < a.n; i += stride) {
        const float v = a.vt[i];
        a.xt[i]       = acc >= 0 ? a.xnext[i] : a.xt[i] - v * a.dt;
        if (a.hist >= 1) {
            a.prev2[i] = a.prev[i];
        }
        a.prev[i] = v;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        if (a.hist == 0) {
            a.status[0] = 0u;
            a.status[1] = 0u;
            a.status[2] = 0u;
        } else {
            a.status[0] += acc < 0 ? 1u : 0u;
            a.status[2] = acc >= 0 ? (uint32_t) a.att_deg[acc] : 0u;
        }
    }
}

int launch_stork4(const StorkArgs & a, const StorkPlan * plans, hipStream_t s) {
    if (a.n == 0) {
        return MI_OK;
    }
    const uint32_t blocks = (uint32_t) std::min<uint64_t>((a.n + 1023) / 1024, 2048);
    if (a.hist > 0) {
        const uint32_t nblk = (uint32_t) std::min<uint64_t>((a.n + 1023) / 1024, STORK_STAT_BLOCKS);
        MI_LAUNCH(k_stork_stats, dim3(nblk), dim3(256), 0, s, a);
        for (int q = 0; q < a.n_attempts; ++q) {
            MI_LAUNCH(k_stork_attempt, dim3(blocks), dim3(256), 0, s, a, plans[q], nblk);
        }
    }
    MI_LAUNCH(k_stork_commit, dim3(blocks), dim3(256), 0, s, a);
    return MI_OK;
}

// ---- DCW (dit-sampler.h:613-667, dwt-haar.h) ---------------------------------
// One thread per (sample, frame pair, channel): denoised = xt - vt * t_next for
// both frames, the Haar analysis of xt and denoised (zero-padded odd tail),
// the band correction x_band += s (x_band - y_band), then the synthesis back
// into the two frames. Pixel mode: xt += s (xt - denoised) per element.
__global__ void __launch_bounds__(256) k_dcw(const DcwArgs a) {
    constexpr float K  = 0.70710678118654752440f;
    const uint32_t  tl = (a.t + 1) / 2;
    const uint64_t  i  = (uint64_t) blockIdx.x * 256u + threadIdx.x;
    if (a.pix) {
        if (i >= (uint64_t) a.n * a.t * a.oc) {
            return;
        }
        const float x = a.xt[i], d = x - a.vt[i] * a.t_next;
        a.xt[i]       = x + a.lo_s * (x - d);
        return;
    }
    if (i >= (uint64_t) a.n * tl * a.oc) {
        return;
    }
    const uint32_t c  = (uint32_t) (i % a.oc);
    const uint64_t r  = i / a.oc;  // sample * tl + pair
    const uint32_t l  = (uint32_t) (r % tl);
    const uint64_t b  = r / tl;
    const uint64_t i0 = (b * a.t + 2u * l) * a.oc + c;
    const bool     two = 2u * l + 1u < a.t;
    const float    x0 = a.xt[i0], d0 = x0 - a.vt[i0] * a.t_next;
    float          xl, xh, yl, yh, x1 = 0.0f;
    if (two) {
        x1             = a.xt[i0 + a.oc];
        const float d1 = x1 - a.vt[i0 + a.oc] * a.t_next;
        xl             = (x0 + x1) * K;
        xh             = (x0 - x1) * K;
        yl             = (d0 + d1) * K;
        yh             = (d0 - d1) * K;
    } else {
        xl = x0 * K;
        xh = x0 * K;
        yl = d0 * K;
        yh = d0 * K;
    }
    if (a.lo_s != 0.0f) {
        xl = xl + a.lo_s * (xl - yl);
    }
    if (a.hi_s != 0.0f) {
        xh = xh + a.hi_s * (xh - yh);
    }
    a.xt[i0] = (xl + xh) * K;
    if (two) {
        a.xt[i0 + a.oc] = (xl - xh) * K;
    }
}

int launch_dcw(const DcwArgs & a, hipStream_t s) {
    const uint64_t work = a.pix ? (uint64_t) a.n * a.t * a.oc : (uint64_t) a.n * ((a.t + 1) / 2) * a.oc;
    if (work == 0) {
        return MI_OK;
    }
    MI_LAUNCH(k_dcw, dim3((uint32_t) ((work + 255) / 256)), dim3(256), 0, s, a);
    return MI_OK;
}

int launch_apg(const ApgArgs & a, hipStream_t s) {
    if (a.n == 0 || a.t == 0 || a.oc == 0) {
        return MI_OK;
    }
    const uint32_t nph = 1024 / a.oc;
    const size_t   lds = (size_t) (3 * nph * a.oc + 3 * a.oc) * sizeof(double);
    MI_LAUNCH(k_apg, dim3(a.n), dim3(nph * a.oc), lds, s, a);
    return MI_OK;
}

int launch_flow_step(const FlowArgs & a, hipStream_t s) {
    if (a.n == 0) {
        return MI_OK;
    }
    MI_LAUNCH(k_flow_step, dim3((uint32_t) ((a.n + 255) / 256)), dim3(256), 0, s, a);
    return MI_OK;
}

}  // namespace mi
