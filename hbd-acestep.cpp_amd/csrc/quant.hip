// quant.hip -- ggml_cpy into KV caches: F32/BF16/F16 -> Q8_0 / F16 / BF16 / F32,
// as a plain strided copy (mi_cpy) or as a batched scatter at per-sequence
// slot offsets (mi_kv_store).
//
// Reference: the F16 KV writes at qwen3-lm.h:396-406 (prefill) and 682-703
// (one cpy node per sequence per K/V per layer in batched decode), and the
// Q8_0 KV writes at songgen-lelm-gen.h:254-265, 548-562.
//
// Q8_0 block quantizer, two ggml variants (bit-exact with each):
//   CPU_X86 (ggml-cpu x86 from_float): amax = max|x|, d = amax/127,
//            id = amax ? 127/amax : 0, q = round-half-even(x*id)
//   REF     (quantize_row_q8_0_ref):   d = amax/127, id = d ? 1/d : 0,
//            q = roundf(x*id)  (half away from zero)
// d is stored as fp16, round to nearest even. Divisions are IEEE
// correctly rounded (the library is not built with fast-math).
//
// Layout: 8 lanes per 32-element block, 4 elements per lane; amax reduced
// with DPP inside the 8 lanes. K and V go in one launch.
#include "launch.h"

namespace mi {

__device__ __forceinline__ float round_half_away(float v) {
    const float t = __builtin_truncf(v);
    return fabsf(v - t) >= 0.5f ? t + __builtin_copysignf(1.0f, v) : t;
}

template <int TI> __device__ __forceinline__ void load4(const char * p, float * f);

template <> __device__ __forceinline__ void load4<MI_TYPE_F32>(const char * p, float * f) {
    unpack16<MI_TYPE_F32>(ld16(p), f);
}

template <> __device__ __forceinline__ void load4<MI_TYPE_BF16>(const char * p, float * f) {
    const uint2 w = *(const uint2 *) p;
    f[0]          = bf16_lo(w.x);
    f[1]          = bf16_hi(w.x);
    f[2]          = bf16_lo(w.y);
    f[3]          = bf16_hi(w.y);
}

template <> __device__ __forceinline__ void load4<MI_TYPE_F16>(const char * p, float * f) {
    const uint2 w = *(const uint2 *) p;
    f[0]          = f16_lo(w.x);
    f[1]          = f16_hi(w.x);
    f[2]          = f16_lo(w.y);
    f[3]          = f16_hi(w.y);
}

// destination row for source row `row`; nullptr when the slot is invalid
__device__ __forceinline__ char * dst_row(const RowCopy & R, uint32_t row, bool & bad) {
    bad = false;
    if (!R.kv) {
        return R.dst + R.dr.off(row);
    }
    const uint32_t i3   = R.d12.div(row);
    const uint32_t rem  = row - i3 * (R.ne1 * R.ne2);
    const uint32_t i2   = R.d1.div(rem);
    const uint32_t i1   = rem - i2 * R.ne1;
    const int64_t  slot = (int64_t) R.pos0[i3] + i2;
    const int64_t  set  = R.sets ? (int64_t) R.sets[i3] : (int64_t) i3;
    if (slot < 0 || slot >= R.max_seq || set < 0 || set >= R.n_sets) {
        bad = true;
        return nullptr;
    }
    return R.dst + slot * R.cnb1 + (int64_t) i1 * R.cnb2 + set * R.cnb3;
}

template <int TI, int TO, int ROUND>
__global__ void __launch_bounds__(256) k_row_copy(const RowCopy K, const RowCopy V, uint32_t nbk, uint32_t total,
                                                  uint32_t nbpr, FastDiv dnbpr) {
    constexpr int  EI  = TT<TI>::ES;
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t blk = gid >> 3;
    const int      sub = gid & 7;
    if (blk >= total) {
        return;
    }
    const bool      isv = blk >= nbk;
    const RowCopy & R   = isv ? V : K;
    const uint32_t  b2  = isv ? blk - nbk : blk;
    const uint32_t  row = dnbpr.div(b2);
    const uint32_t  bi  = b2 - row * nbpr;
    bool            bad;
    char *          drow = dst_row(R, row, bad);
    if (bad) {
        if (sub == 0 && bi == 0 && R.d_err) {
            atomicAdd(R.d_err, 1);
        }
        return;
    }
    const int    e0 = (int) bi * 32 + sub * 4;
    float        f[4];
    load4<TI>(R.src + R.sr.off(row) + (size_t) e0 * EI, f);
    if constexpr (TO == MI_TYPE_Q8_0) {
        float amax = fmaxf(fmaxf(fabsf(f[0]), fabsf(f[1])), fmaxf(fabsf(f[2]), fabsf(f[3])));
        amax       = group_max<8>(amax);
        const float d = amax / 127.0f;
        float       id;
        if constexpr (ROUND == MI_Q8_0_REF) {
            id = d != 0.0f ? 1.0f / d : 0.0f;
        } else {
            id = amax != 0.0f ? 127.0f / amax : 0.0f;
        }
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = f[e] * id;
            float       q;
            if constexpr (ROUND == MI_Q8_0_REF) {
                q = round_half_away(v);
            } else {
                q = __builtin_rintf(v);
                q = fminf(fmaxf(q, -128.0f), 127.0f);
            }
            packed |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        char * bp = drow + (size_t) bi * 34;
        uint16_t * qp = (uint16_t *) (bp + 2 + sub * 4);
        qp[0]         = (uint16_t) (packed & 0xffffu);
        qp[1]         = (uint16_t) (packed >> 16);
        if (sub == 0) {
            *(uint16_t *) bp = f32_to_f16_bits(d);
        }
    } else if constexpr (TO == MI_TYPE_F32) {
        st16(drow + (size_t) e0 * 4, pack16<MI_TYPE_F32>(f));
    } else {
        store_vec<TO, 4>(drow + (size_t) e0 * 2, f);
    }
}

// Generic: one thread per destination block (Q8_0) or element (others),
// any alignment / row length (Q8_0 still needs whole blocks).
template <int TI, int TO, int ROUND>
__global__ void __launch_bounds__(256) k_row_copy_generic(const RowCopy K, const RowCopy V, uint64_t nk,
                                                          uint64_t total, int per_row) {
    constexpr int EI = TT<TI>::ES;
    for (uint64_t g = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x; g < total;
         g += (uint64_t) gridDim.x * blockDim.x) {
        const bool      isv = g >= nk;
        const RowCopy & R   = isv ? V : K;
        const uint64_t  g2  = isv ? g - nk : g;
        const uint32_t  row = (uint32_t) (g2 / per_row);
        const int       c   = (int) (g2 - (uint64_t) row * per_row);
        bool            bad;
        char *          drow = dst_row(R, row, bad);
        if (bad) {
            if (c == 0 && R.d_err) {
                atomicAdd(R.d_err, 1);
            }
            continue;
        }
        const char * srow = R.src + R.sr.off(row);
        if constexpr (TO == MI_TYPE_Q8_0) {
            float x[32];
            float amax = 0.0f;
            for (int e = 0; e < 32; ++e) {
                x[e] = load_elem<TI>(srow + (size_t) (c * 32 + e) * EI);
                amax = fmaxf(amax, fabsf(x[e]));
            }
            const float d  = amax / 127.0f;
            const float id = ROUND == MI_Q8_0_REF ? (d != 0.0f ? 1.0f / d : 0.0f) : (amax != 0.0f ? 127.0f / amax : 0.0f);
            char *      bp = drow + (size_t) c * 34;
            for (int e = 0; e < 32; ++e) {
                const float v = x[e] * id;
                float       q = ROUND == MI_Q8_0_REF ? round_half_away(v) : fminf(fmaxf(__builtin_rintf(v), -128.0f), 127.0f);
                bp[2 + e]     = (char) (int8_t) (int32_t) q;
            }
            const uint16_t dh = f32_to_f16_bits(d);
            bp[0]             = (char) (dh & 0xff);
            bp[1]             = (char) (dh >> 8);
        } else {
            const float v = load_elem<TI>(srow + (size_t) c * EI);
            store_elem<TO>(drow + (size_t) c * TT<TO>::ES, v);
        }
    }
}

template <int TI, int TO, int ROUND>
static int launch_k(const RowCopy & K, const RowCopy * V, bool fast, hipStream_t s) {
    const RowCopy & Vr = V ? *V : K;
    if (fast) {
        const uint32_t nbpr  = (uint32_t) (K.ne0 / 32);
        const uint32_t nbk   = K.rows * nbpr;
        const uint32_t total = nbk + (V ? V->rows * nbpr : 0);
        const uint32_t grid  = (total * 8 + 255) / 256;
        hipLaunchKernelGGL((k_row_copy<TI, TO, ROUND>), dim3(grid), dim3(256), 0, s, K, Vr, nbk, total, nbpr,
                           FastDiv(nbpr));
        return MI_OK;
    }
    const int      per_row = TO == MI_TYPE_Q8_0 ? K.ne0 / 32 : K.ne0;
    const uint64_t nk      = (uint64_t) K.rows * per_row;
    const uint64_t total   = nk + (V ? (uint64_t) V->rows * per_row : 0);
    uint64_t       grid    = (total + 255) / 256;
    const uint64_t cap     = (uint64_t) num_cus() * 32;
    grid                   = grid > cap ? cap : (grid ? grid : 1);
    hipLaunchKernelGGL((k_row_copy_generic<TI, TO, ROUND>), dim3((uint32_t) grid), dim3(256), 0, s, K, Vr, nk, total,
                       per_row);
    return MI_OK;
}

template <int TI, int TO>
static int launch_r(const RowCopy & K, const RowCopy * V, int rounding, bool fast, hipStream_t s) {
    if (TO == MI_TYPE_Q8_0 && rounding == MI_Q8_0_REF) {
        return launch_k<TI, TO, MI_Q8_0_REF>(K, V, fast, s);
    }
    return launch_k<TI, TO, MI_Q8_0_CPU_X86>(K, V, fast, s);
}

template <int TI>
static int launch_ti(const RowCopy & K, const RowCopy * V, int tout, int rounding, bool fast, hipStream_t s) {
    switch (tout) {
        case MI_TYPE_Q8_0:
            return launch_r<TI, MI_TYPE_Q8_0>(K, V, rounding, fast, s);
        case MI_TYPE_F32:
            return launch_r<TI, MI_TYPE_F32>(K, V, rounding, fast, s);
        case MI_TYPE_BF16:
            return launch_r<TI, MI_TYPE_BF16>(K, V, rounding, fast, s);
        default:
            return launch_r<TI, MI_TYPE_F16>(K, V, rounding, fast, s);
    }
}

static bool row_aligned(const RowCopy & R, int tin, int tout) {
    const int sa = tin == MI_TYPE_F32 ? 16 : 8;  // 4-element source loads
    if (!aligned(R.src, sa) || R.sr.s1 % sa || R.sr.s2 % sa || R.sr.s3 % sa) {
        return false;
    }
    if (tout == MI_TYPE_Q8_0) {  // 16-bit stores into 34-byte blocks
        return aligned(R.dst, 2) && (R.kv ? (R.cnb1 % 2 == 0 && R.cnb2 % 2 == 0 && R.cnb3 % 2 == 0)
                                          : (R.dr.s1 % 2 == 0 && R.dr.s2 % 2 == 0 && R.dr.s3 % 2 == 0));
    }
    const int da = tout == MI_TYPE_F32 ? 16 : 8;
    return aligned(R.dst, da) && (R.kv ? (R.cnb1 % da == 0 && R.cnb2 % da == 0 && R.cnb3 % da == 0)
                                       : (R.dr.s1 % da == 0 && R.dr.s2 % da == 0 && R.dr.s3 % da == 0));
}

int launch_row_copy(const RowCopy & K, const RowCopy * V, int tin, int tout, int rounding, hipStream_t s) {
    if (K.rows == 0 || K.ne0 == 0) {
        return MI_OK;
    }
    bool fast = K.ne0 % 32 == 0 && row_aligned(K, tin, tout) && (!V || row_aligned(*V, tin, tout));
    fast      = fast && (uint64_t) (K.rows + (V ? V->rows : 0)) * (K.ne0 / 32) * 8 < (1ull << 31);
    switch (tin) {
        case MI_TYPE_F32:
            return launch_ti<MI_TYPE_F32>(K, V, tout, rounding, fast, s);
        case MI_TYPE_BF16:
            return launch_ti<MI_TYPE_BF16>(K, V, tout, rounding, fast, s);
        default:
            return launch_ti<MI_TYPE_F16>(K, V, tout, rounding, fast, s);
    }
}

}  // namespace mi
