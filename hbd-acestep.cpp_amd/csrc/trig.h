// trig.h -- single-precision sin/cos for rotary angles, usable on the device
// and (for testing) on the host.
//
// Method: Cody-Waite reduction x = k*(pi/2) + r with pi/2 split into three
// fp32 parts (P1 + P2 + P3; k*P1 is exact inside the fma and x - k*P1 is
// exact), then the Taylor series of sin and cos, evaluated by Horner in fp32,
// and the quadrant k mod 4 picks/negates the two results:
//   sin r = r + r^3 (-1/3! + r^2 (1/5! + r^2 (-1/7! + r^2/9!)))
//   cos r = 1 + r^2 (-1/2! + r^2 (1/4! + r^2 (-1/6! + r^2 (1/8! - r^2/10!))))
// For |x| < 2^20 the fp32 product x*(2/pi) is off by < 0.05, so |r| < 0.87
// and the truncation terms stay below 1e-8. Measured on the host over every
// third float in (-2^20, 2^20): max |error| 7.2e-8 against double-precision
// sin/cos (glibc sinf/cosf: 3.3e-8). Rotary angles are pos * theta_scale^i,
// so |x| < 2^20 covers positions below 2^20; larger or non-finite arguments
// take the math library's sincosf.
#pragma once

#if defined(__HIPCC__)
#define MI_HD    __host__ __device__ __forceinline__
#define MI_HD_NI static __host__ __device__ __attribute__((noinline))
#else
#include <math.h>
#define MI_HD    static inline
#define MI_HD_NI static
#endif

namespace mi {

struct float2_t {
    float s, c;
};

// |x| >= 2^20 or non-finite: the math library. Kept out of line so that the
// fast path does not carry (or speculatively execute) its large-argument
// reduction; it returns by value (no pointer into private memory).
MI_HD_NI float2_t sincos_rot_big(float x) {
    float2_t r;
#if defined(__HIP_DEVICE_COMPILE__)
    sincosf(x, &r.s, &r.c);
#else
    r.s = sinf(x);
    r.c = cosf(x);
#endif
    return r;
}

MI_HD void sincos_rot(float x, float * sp, float * cp) {
    const float ax = __builtin_fabsf(x);
    if (!(ax < 1048576.0f)) {  // |x| >= 2^20 or NaN
        const float2_t r = sincos_rot_big(x);
        *sp              = r.s;
        *cp              = r.c;
        return;
    }
    const float TWO_OVER_PI = 0.636619746685028076171875f;           // fp32(2/pi)
    const float P1          = 1.57079637050628662109375f;             // fp32(pi/2)
    const float P2          = -4.37113882867379300296306610107421875e-08f;  // fp32(pi/2 - P1)
    const float P3          = -1.71512451000588189e-15f;             // fp32(pi/2 - P1 - P2)
    const float k           = __builtin_rintf(x * TWO_OVER_PI);
    float       r           = __builtin_fmaf(-k, P1, x);
    r                       = __builtin_fmaf(-k, P2, r);
    r                       = __builtin_fmaf(-k, P3, r);
    const float r2          = r * r;
    float       ps          = 1.0f / 362880.0f;
    ps                      = __builtin_fmaf(ps, r2, -1.0f / 5040.0f);
    ps                      = __builtin_fmaf(ps, r2, 1.0f / 120.0f);
    ps                      = __builtin_fmaf(ps, r2, -1.0f / 6.0f);
    const float sr          = __builtin_fmaf(ps * r2, r, r);
    float       pc          = -1.0f / 3628800.0f;
    pc                      = __builtin_fmaf(pc, r2, 1.0f / 40320.0f);
    pc                      = __builtin_fmaf(pc, r2, -1.0f / 720.0f);
    pc                      = __builtin_fmaf(pc, r2, 1.0f / 24.0f);
    pc                      = __builtin_fmaf(pc, r2, -0.5f);
    const float cr          = __builtin_fmaf(pc, r2, 1.0f);
    // x = k*pi/2 + r: quadrant q = k mod 4 (two's complement for k < 0)
    //   q: 0 -> ( s,  c)   1 -> ( c, -s)   2 -> (-s, -c)   3 -> (-c,  s)
    const int   q           = (int) k;
    const float s           = (q & 1) ? cr : sr;
    const float c           = (q & 1) ? sr : cr;
    *sp                     = x == 0.0f ? x : ((q & 2) ? -s : s);  // sin(-0) = -0
    *cp                     = ((q + 1) & 2) ? -c : c;
}

}  // namespace mi
