// common.h -- shared device helpers for the gfx950 per-layer op kernels.
//
// Conventions used by every kernel in this library:
//  * wave64; a "vector" is 16 bytes (4 x f32 or 8 x bf16/f16) so each lane
//    issues 128-bit loads/stores;
//  * all arithmetic in fp32, in the order the ggml nodes apply it; the
//    library is built with -ffp-contract=off so no multiply/add pair is
//    silently fused (fused multiply-adds appear only as explicit fmaf);
//  * cross-lane reductions use DPP inside a 16-lane row and bpermute
//    shuffles across rows.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mi_ops.h"
#include "validate.h"

namespace mi {

constexpr int WAVE = 64;

// ---------------------------------------------------------------------------
// fast unsigned division by a run-time constant (n < 2^31): q = (mulhi(n,m)+n) >> s
// ---------------------------------------------------------------------------
struct FastDiv {
    uint32_t d, m, s;

    __host__ __device__ FastDiv() : d(1), m(1), s(0) {}

    __host__ explicit FastDiv(uint32_t dd) {
        d = dd ? dd : 1;
        s = 0;
        while ((1ull << s) < d) {
            ++s;
        }
        const uint64_t one = 1;
        m                  = (uint32_t) (((one << 32) * ((one << s) - d)) / d + 1);
    }

    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const {
#if defined(__HIP_DEVICE_COMPILE__)
        const uint32_t t = __umulhi(n, m);
#else
        const uint32_t t = (uint32_t) (((uint64_t) n * m) >> 32);
#endif
        return (t + n) >> s;
    }
};

// ---------------------------------------------------------------------------
// element conversions
// ---------------------------------------------------------------------------
typedef float    f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16   bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t w) {
    return __uint_as_float(w << 16);
}

__device__ __forceinline__ float bf16_hi(uint32_t w) {
    return __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ float f16_lo(uint32_t w) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) (w & 0xffffu));
}

__device__ __forceinline__ float f16_hi(uint32_t w) {
    return (float) __builtin_bit_cast(_Float16, (uint16_t) (w >> 16));
}

// round-to-nearest-even packs (v_cvt_pk_bf16_f32 on gfx950)
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    f32x2 v = { a, b };
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    f32x2 v = { a, b };
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
}

__device__ __forceinline__ uint16_t f32_to_f16_bits(float a) {
    return __builtin_bit_cast(uint16_t, (_Float16) a);
}

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float a) {
    return __builtin_bit_cast(uint16_t, (__bf16) a);
}

// Type traits for activation storage types.
template <int T> struct TT;

template <> struct TT<MI_TYPE_F32> {
    static constexpr int ES  = 4;
    static constexpr int VEC = 4;
};

template <> struct TT<MI_TYPE_BF16> {
    static constexpr int ES  = 2;
    static constexpr int VEC = 8;
};

template <> struct TT<MI_TYPE_F16> {
    static constexpr int ES  = 2;
    static constexpr int VEC = 8;
};

// 16-byte vector <-> floats
template <int T> __device__ __forceinline__ void unpack16(const uint4 & v, float * f);

template <> __device__ __forceinline__ void unpack16<MI_TYPE_F32>(const uint4 & v, float * f) {
    f[0] = __uint_as_float(v.x);
    f[1] = __uint_as_float(v.y);
    f[2] = __uint_as_float(v.z);
    f[3] = __uint_as_float(v.w);
}

template <> __device__ __forceinline__ void unpack16<MI_TYPE_BF16>(const uint4 & v, float * f) {
    f[0] = bf16_lo(v.x);
    f[1] = bf16_hi(v.x);
    f[2] = bf16_lo(v.y);
    f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z);
    f[5] = bf16_hi(v.z);
    f[6] = bf16_lo(v.w);
    f[7] = bf16_hi(v.w);
}

template <> __device__ __forceinline__ void unpack16<MI_TYPE_F16>(const uint4 & v, float * f) {
    f[0] = f16_lo(v.x);
    f[1] = f16_hi(v.x);
    f[2] = f16_lo(v.y);
    f[3] = f16_hi(v.y);
    f[4] = f16_lo(v.z);
    f[5] = f16_hi(v.z);
    f[6] = f16_lo(v.w);
    f[7] = f16_hi(v.w);
}

// Pack VEC_OUT floats into the output storage; returns the packed words in
// a uint4 (F32: 4 floats; BF16/F16: 8 floats).
template <int T> __device__ __forceinline__ uint4 pack16(const float * f);

template <> __device__ __forceinline__ uint4 pack16<MI_TYPE_F32>(const float * f) {
    return make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
}

template <> __device__ __forceinline__ uint4 pack16<MI_TYPE_BF16>(const float * f) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
}

template <> __device__ __forceinline__ uint4 pack16<MI_TYPE_F16>(const float * f) {
    return make_uint4(pack_f16x2(f[0], f[1]), pack_f16x2(f[2], f[3]), pack_f16x2(f[4], f[5]), pack_f16x2(f[6], f[7]));
}

// Scalar element access (generic paths).
template <int T> __device__ __forceinline__ float load_elem(const char * p);

template <> __device__ __forceinline__ float load_elem<MI_TYPE_F32>(const char * p) {
    return *(const float *) p;
}

template <> __device__ __forceinline__ float load_elem<MI_TYPE_BF16>(const char * p) {
    return __uint_as_float((uint32_t) (*(const uint16_t *) p) << 16);
}

template <> __device__ __forceinline__ float load_elem<MI_TYPE_F16>(const char * p) {
    return (float) __builtin_bit_cast(_Float16, *(const uint16_t *) p);
}

template <int T> __device__ __forceinline__ void store_elem(char * p, float v);

template <> __device__ __forceinline__ void store_elem<MI_TYPE_F32>(char * p, float v) {
    *(float *) p = v;
}

template <> __device__ __forceinline__ void store_elem<MI_TYPE_BF16>(char * p, float v) {
    *(uint16_t *) p = f32_to_bf16_bits(v);
}

template <> __device__ __forceinline__ void store_elem<MI_TYPE_F16>(char * p, float v) {
    *(uint16_t *) p = f32_to_f16_bits(v);
}

// Streaming (activation) loads/stores. MI_NT_LD / MI_NT_ST select the
// non-temporal cache policy (each activation byte is touched once).
#ifndef MI_NT_LD
#define MI_NT_LD 1
#endif
#ifndef MI_NT_ST
#define MI_NT_ST 1
#endif
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// A wave-uniform load of data the kernel never writes, through the scalar
// memory path: it is counted apart from the vector loads, so waiting for it
// does not wait for the vector loads issued before it.
__device__ __forceinline__ int32_t ld_scalar_i32(const int32_t * p, int64_t i) {
    return ((const __attribute__((address_space(4))) int32_t *) p)[i];
}

__device__ __forceinline__ uint4 ld16(const char * p) {
#if MI_NT_LD
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *) p);
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return *(const uint4 *) p;
#endif
}

__device__ __forceinline__ void st16(char * p, const uint4 & v) {
#if MI_NT_ST
    const u32x4 w = { v.x, v.y, v.z, v.w };
    __builtin_nontemporal_store(w, (u32x4 *) p);
#else
    *(uint4 *) p = v;
#endif
}

__device__ __forceinline__ void st8(char * p, const uint2 & v) {
#if MI_NT_ST
    const u32x2 w = { v.x, v.y };
    __builtin_nontemporal_store(w, (u32x2 *) p);
#else
    *(uint2 *) p = v;
#endif
}

// round an fp32 value to the storage type and back (identity for F32)
template <int T> __device__ __forceinline__ float round_to(float v) {
    if constexpr (T == MI_TYPE_BF16) {
        return __uint_as_float((uint32_t) f32_to_bf16_bits(v) << 16);
    } else if constexpr (T == MI_TYPE_F16) {
        return (float) __builtin_bit_cast(_Float16, f32_to_f16_bits(v));
    } else {
        return v;
    }
}

// ---------------------------------------------------------------------------
// Q8_0 block quantizer pieces (ggml's two variants, see quant.hip)
// ---------------------------------------------------------------------------
__device__ __forceinline__ float round_half_away(float v) {
    const float t = __builtin_truncf(v);
    return fabsf(v - t) >= 0.5f ? t + __builtin_copysignf(1.0f, v) : t;
}

// d = amax / 127: amax * RN(1/127) corrected by one fma, equal to the IEEE
// quotient for every non-negative float (checked exhaustively on the host)
__device__ __forceinline__ float div127(float amax) {
    constexpr float C  = 1.0f / 127.0f;
    const float     q0 = amax * C;
    const float     r  = __builtin_fmaf(-q0, 127.0f, amax);
    return __builtin_fmaf(r, C, q0);
}

// An optimization barrier on a register quad: its value is treated as changed,
// so values derived from it before are recomputed after, not kept live.
__device__ __forceinline__ void opaque(uint4 & v) {
    asm volatile("" : "+v"(v.x), "+v"(v.y), "+v"(v.z), "+v"(v.w));
}

// ---------------------------------------------------------------------------
// cross-lane reductions
// ---------------------------------------------------------------------------
// DPP controls (gfx9): quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141 (lane i <-> 7-i in each 8), row_mirror = 0x140
// (lane i <-> 15-i in each 16).
template <int CTRL> __device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <int CTRL> __device__ __forceinline__ double dpp_d(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int) __double2loint(v), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int) __double2hiint(v), CTRL, 0xf, 0xf, false);
    return __hiloint2double(hi, lo);
}

// Sum over aligned groups of L lanes (L = 1..64, power of two). Every lane of
// a group ends with the bit-identical total (each step adds a commutative pair).
template <int L> __device__ __forceinline__ double group_sum(double v) {
    if constexpr (L >= 2) {
        v += dpp_d<0xB1>(v);
    }
    if constexpr (L >= 4) {
        v += dpp_d<0x4E>(v);
    }
    if constexpr (L >= 8) {
        v += dpp_d<0x141>(v);
    }
    if constexpr (L >= 16) {
        v += dpp_d<0x140>(v);
    }
    if constexpr (L >= 32) {
        v += __shfl_xor(v, 16, 64);
    }
    if constexpr (L >= 64) {
        v += __shfl_xor(v, 32, 64);
    }
    return v;
}

template <int L> __device__ __forceinline__ float group_sum(float v) {
    if constexpr (L >= 2) {
        v += dpp_f<0xB1>(v);
    }
    if constexpr (L >= 4) {
        v += dpp_f<0x4E>(v);
    }
    if constexpr (L >= 8) {
        v += dpp_f<0x141>(v);
    }
    if constexpr (L >= 16) {
        v += dpp_f<0x140>(v);
    }
    if constexpr (L >= 32) {
        v += __shfl_xor(v, 16, 64);
    }
    if constexpr (L >= 64) {
        v += __shfl_xor(v, 32, 64);
    }
    return v;
}

// silu(x) = x / (1 + e^-x) for SwiGLU (glu.hip) and the SwiGLU prologue of the
// Q8_0 product (matmul.hip): e^-x as v_exp_f32 (2^t) on t = -x*log2(e), with the
// rounding error of that product recovered by an fma and folded back in first
// order, so e^-x is good to ~1 ulp over the finite range; the quotient is
// x * v_rcp_f32(1 + e^-x).
#ifndef MI_SILU_CORR
#define MI_SILU_CORR 1  // recover the rounding error of -x*log2(e) (first order)
#endif

__device__ __forceinline__ float silu_f(float x) {
    constexpr float LOG2E = 1.44269504088896340736f;  // rounded log2(e)
    const float     t     = -x * LOG2E;
#if MI_SILU_CORR
    constexpr float LOG2E_LO = 1.925963033500011e-08f;  // log2(e) - LOG2E
    constexpr float LN2      = 0.693147180559945309417f;
    const float     terr     = __builtin_fmaf(-x, LOG2E_LO, __builtin_fmaf(-x, LOG2E, -t));
    const float     e0       = __builtin_amdgcn_exp2f(t);
    // first-order correction only where 2^t is finite and t finite (for t = -inf
    // the residual is +inf and 0*inf would give NaN)
    const float     e        = __builtin_fabsf(t) < 128.0f ? __builtin_fmaf(e0, terr * LN2, e0) : e0;
#else
    const float e = __builtin_amdgcn_exp2f(t);
#endif
    const float d = 1.0f + e;
    return x * __builtin_amdgcn_rcpf(d);
}

template <int L> __device__ __forceinline__ float group_max(float v) {
    if constexpr (L >= 2) {
        v = fmaxf(v, dpp_f<0xB1>(v));
    }
    if constexpr (L >= 4) {
        v = fmaxf(v, dpp_f<0x4E>(v));
    }
    if constexpr (L >= 8) {
        v = fmaxf(v, dpp_f<0x141>(v));
    }
    if constexpr (L >= 16) {
        v = fmaxf(v, dpp_f<0x140>(v));
    }
    if constexpr (L >= 32) {
        v = fmaxf(v, __shfl_xor(v, 16, 64));
    }
    if constexpr (L >= 64) {
        v = fmaxf(v, __shfl_xor(v, 32, 64));
    }
    return v;
}

// cos/sin/exp/log of an fp32 argument evaluated in double and rounded once to
// fp32: correctly rounded except in vanishingly rare cases, which is what
// glibc's cosf/sinf/expf/logf (called by ggml-cpu) deliver as well, so both
// sides agree in nearly every value instead of differing by device-libm ulps.
__device__ __forceinline__ void sincos_f32(float x, float * s, float * c) {
    double sd, cd;
    sincos((double) x, &sd, &cd);
    *s = (float) sd;
    *c = (float) cd;
}

__device__ __forceinline__ float exp_f32(float x) {
    return (float) exp((double) x);
}

__device__ __forceinline__ float log_f32(float x) {
    return (float) log((double) x);
}

// ggml-cpu rms_norm scale from the double sum of float squares:
// mean = (float)(sum / n), scale = 1.0f / sqrtf(mean + eps). For n a power of
// two, sum / n == sum * (1/n) exactly (a sum of float squares is never a
// double subnormal), so the division becomes a multiply.
// ggml_clamp: MAX(MIN(v, hi), lo) with C's comparison macros (a NaN becomes hi)
__device__ __forceinline__ float clamp_ggml(float v, float lo, float hi) {
    const float t = v < hi ? v : hi;
    return t > lo ? t : lo;
}

// RMSNorm sum of squares. F32 activations: ggml's arithmetic, the float
// square summed in double. BF16/F16 activations: fp32 accumulation (one fma
// per element), the arithmetic the bf16 bar is stated for; it keeps the
// row scale within a few fp32 ulp of the double sum.
template <int TI> using sq_t = typename std::conditional<TI == MI_TYPE_F32, double, float>::type;

template <int TI> __device__ __forceinline__ sq_t<TI> sq_acc(sq_t<TI> acc, float x) {
    if constexpr (TI == MI_TYPE_F32) {
        return acc + (double) (x * x);
    } else {
        return __builtin_fmaf(x, x, acc);
    }
}

__device__ __forceinline__ float rms_scale(float sum, int n, float eps) {
    const float mean = (n & (n - 1)) == 0 ? sum * (1.0f / (float) n) : sum / (float) n;
    return 1.0f / sqrtf(mean + eps);
}

__device__ __forceinline__ float rms_scale(double sum, int n, float eps) {
    const float mean = (n & (n - 1)) == 0 ? (float) (sum * (1.0 / (double) n)) : (float) (sum / (double) n);
    return 1.0f / sqrtf(mean + eps);
}

// ---------------------------------------------------------------------------
// host-side descriptor helpers
// ---------------------------------------------------------------------------
inline int type_size(int t) {
    switch (t) {
        case MI_TYPE_F32:
        case MI_TYPE_I32:
            return 4;
        case MI_TYPE_F16:
        case MI_TYPE_BF16:
            return 2;
        case MI_TYPE_Q8_0:
            return 34;
        default:
            return 0;
    }
}

inline int blck_size(int t) {
    return t == MI_TYPE_Q8_0 ? 32 : 1;
}

inline bool is_act(int t) {
    return t == MI_TYPE_F32 || t == MI_TYPE_BF16 || t == MI_TYPE_F16;
}

inline int64_t nelements(const mi_tensor & t) {
    return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3];
}

inline int64_t nrows(const mi_tensor & t) {
    return t.ne[1] * t.ne[2] * t.ne[3];
}

inline bool same_shape(const mi_tensor & a, const mi_tensor & b) {
    return a.ne[0] == b.ne[0] && a.ne[1] == b.ne[1] && a.ne[2] == b.ne[2] && a.ne[3] == b.ne[3];
}

// a contiguous F32 vector of n elements (as a ggml [n] tensor)
inline bool is_vec_f32(const mi_tensor & t, int64_t n) {
    return t.type == MI_TYPE_F32 && t.ne[0] == n && t.ne[1] == 1 && t.ne[2] == 1 && t.ne[3] == 1 && t.nb[0] == 4;
}

inline bool aligned(const void * p, size_t a) {
    return ((uintptr_t) p % a) == 0;
}

// Row addressing for [ne0, ne1, ne2, ne3] views: row r -> (i1, i2, i3).
// When the rows are uniformly strided (nb2 == ne1*nb1, nb3 == ne2*nb2, the
// usual case) the offset is one multiply.
struct Rows3 {
    FastDiv  d1, d12;   // ne1, ne1*ne2
    uint32_t ne1, ne2;
    int64_t  s1, s2, s3; // byte strides
    int      uni;       // rows uniformly strided by s1

    __device__ __forceinline__ int64_t off(uint32_t r) const {
        if (uni) {
            return (int64_t) r * s1;
        }
        const uint32_t i3  = d12.div(r);
        const uint32_t rem = r - i3 * (ne1 * ne2);
        const uint32_t i2  = d1.div(rem);
        const uint32_t i1  = rem - i2 * ne1;
        return (int64_t) i1 * s1 + (int64_t) i2 * s2 + (int64_t) i3 * s3;
    }
};

inline Rows3 make_rows3(const mi_tensor & t) {
    Rows3 r;
    r.ne1 = (uint32_t) t.ne[1];
    r.ne2 = (uint32_t) t.ne[2];
    r.d1  = FastDiv((uint32_t) t.ne[1]);
    r.d12 = FastDiv((uint32_t) (t.ne[1] * t.ne[2]));
    r.s1  = (int64_t) t.nb[1];
    r.s2  = (int64_t) t.nb[2];
    r.s3  = (int64_t) t.nb[3];
    // row r sits at r*nb1 iff every used outer stride is the packed one
    r.uni = (t.ne[2] <= 1 || t.nb[2] == t.nb[1] * (uint64_t) t.ne[1]) &&
            (t.ne[3] <= 1 || t.nb[3] == t.nb[1] * (uint64_t) (t.ne[1] * t.ne[2]));
    return r;
}

int num_cus();  // cached per device

}  // namespace mi
