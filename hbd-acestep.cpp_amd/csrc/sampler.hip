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

// solver 0 euler, 1 dpm3m (hist = stored velocities: 0, 1 or 2), 2 final x0
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

int launch_apg(const ApgArgs & a, hipStream_t s) {
    if (a.n == 0 || a.t == 0 || a.oc == 0) {
        return MI_OK;
    }
    const uint32_t nph = 1024 / a.oc;
    const size_t   lds = (size_t) (3 * nph * a.oc + 3 * a.oc) * sizeof(double);
    hipLaunchKernelGGL(k_apg, dim3(a.n), dim3(nph * a.oc), lds, s, a);
    return MI_OK;
}

int launch_flow_step(const FlowArgs & a, hipStream_t s) {
    if (a.n == 0) {
        return MI_OK;
    }
    hipLaunchKernelGGL(k_flow_step, dim3((uint32_t) ((a.n + 255) / 256)), dim3(256), 0, s, a);
    return MI_OK;
}

}  // namespace mi
