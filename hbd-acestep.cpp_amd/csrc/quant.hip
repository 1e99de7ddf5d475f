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
// d is stored as fp16, round to nearest even. 127/amax and 1/d are IEEE
// divisions; d = amax/127 is amax*RN(1/127) corrected by one fma, which
// equals the IEEE quotient for every non-negative float (checked
// exhaustively on the host; the kernels keep f32 denormals).
//
// Q8_0 destinations: 2 lanes per 32-element block, 16 elements (two or four
// 16-byte loads) per lane, amax reduced with one DPP step, so the per-block
// work (row and slot lookup, amax, the divisions, the fp16 scale) is shared
// by 16 elements per lane. F32/F16/BF16 destinations: 4 lanes x 8 elements.
// In the KV store, rows are walked head-major (sequence, head, token), so
// consecutive rows land in consecutive cache slots and a wave's stores cover
// contiguous bytes. K and V go in one launch.
#include "launch.h"

namespace mi {


// 8 consecutive source elements (32 bytes of F32, 16 of BF16/F16), 16-byte aligned
template <int TI> __device__ __forceinline__ void load8(const char * p, float * f) {
    if constexpr (TI == MI_TYPE_F32) {
        unpack16<MI_TYPE_F32>(ld16(p), f);
        unpack16<MI_TYPE_F32>(ld16(p + 16), f + 4);
    } else {
        unpack16<TI>(ld16(p), f);
    }
}

// Work row w -> source row pointer and destination row (nullptr-free: `bad`
// marks an invalid slot or set). Plain copies use the source's row order; KV
// stores walk (sequence i3, head i1, token i2) with the token fastest.
#ifndef MI_KV_HEAD_MAJOR
#define MI_KV_HEAD_MAJOR 1
#endif
#ifndef MI_Q8_LPB
#define MI_Q8_LPB 4  // lanes per 32-element block in the unstaged Q8_0 store (2 or 4)
#endif
#ifndef MI_Q8_LDS
#define MI_Q8_LDS 1  // Q8_0 store through an LDS tile (lane-contiguous source loads)
#endif

// (head i1, token i2, sequence i3) of KV work row w
__device__ __forceinline__ void kv_index(const RowCopy & R, uint32_t w, uint32_t & i1, uint32_t & i2, uint32_t & i3) {
#if MI_KV_HEAD_MAJOR
    const uint32_t q = R.d2.div(w);
    i2               = w - q * R.ne2;
    i3               = R.d1.div(q);
    i1               = q - i3 * R.ne1;
#else
    const uint32_t q = R.d1.div(w);
    i1               = w - q * R.ne1;
    i3               = R.d2.div(q);
    i2               = q - i3 * R.ne2;
#endif
}

// source row of work row w
__device__ __forceinline__ const char * src_ptr(const RowCopy & R, uint32_t w) {
    if (!R.kv) {
        return R.src + R.sr.off(w);
    }
    uint32_t i1, i2, i3;
    kv_index(R, w, i1, i2, i3);
    return R.src + (int64_t) i1 * R.sr.s1 + (int64_t) i2 * R.sr.s2 + (int64_t) i3 * R.sr.s3;
}

// both rows of work row w; `bad` marks an invalid cache slot or set
__device__ __forceinline__ void row_ptrs(const RowCopy & R, uint32_t w, const char *& src, char *& dst, bool & bad) {
    bad = false;
    if (!R.kv) {
        src = R.src + R.sr.off(w);
        dst = R.dst + R.dr.off(w);
        return;
    }
    uint32_t i1, i2, i3;
    kv_index(R, w, i1, i2, i3);
    src                = R.src + (int64_t) i1 * R.sr.s1 + (int64_t) i2 * R.sr.s2 + (int64_t) i3 * R.sr.s3;
    const int64_t slot = (int64_t) R.pos0[i3] + i2;
    const int64_t set  = R.sets ? (int64_t) R.sets[i3] : (int64_t) i3;
    bad                = slot < 0 || slot >= R.max_seq || set < 0 || set >= R.n_sets;
    dst                = R.dst + slot * R.cnb1 + (int64_t) i1 * R.cnb2 + set * R.cnb3;
}


template <int TI, int ROUND>
__global__ void __launch_bounds__(256) k_row_q8(const RowCopy K, const RowCopy V, uint32_t nbk, uint32_t total,
                                                uint32_t nbpr, FastDiv dnbpr) {
    constexpr int  EI  = TT<TI>::ES;
    constexpr int  LPB = MI_Q8_LPB;  // lanes per 32-element block
    constexpr int  EPL = 32 / LPB;   // elements per lane
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t blk = gid / LPB;
    const int      sub = gid % LPB;
    if (blk >= total) {
        return;  // whole lane groups
    }
    const bool      isv = blk >= nbk;
    const RowCopy & R   = isv ? V : K;
    const uint32_t  b2  = isv ? blk - nbk : blk;
    const uint32_t  w   = dnbpr.div(b2);
    const uint32_t  bi  = b2 - w * nbpr;
    const char *    src;
    char *          drow;
    bool            bad;
    row_ptrs(R, w, src, drow, bad);
    float f[EPL];
    {
        constexpr int VV = TT<TI>::VEC;
        const char *  p  = src + (size_t) (bi * 32 + sub * EPL) * EI;  // independent of the slot check
#pragma unroll
        for (int k = 0; k < EPL / VV; ++k) {
            unpack16<TI>(ld16(p + 16 * k), f + VV * k);
        }
    }
    if (bad) {
        if (sub == 0 && bi == 0 && R.d_err) {
            atomicAdd(R.d_err, 1);
        }
        return;  // the whole row's lane groups
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        amax = fmaxf(amax, fabsf(f[e]));
    }
    amax          = group_max<LPB>(amax);
    const float d = div127(amax);
    float       id;
    if constexpr (ROUND == MI_Q8_0_REF) {
        id = d != 0.0f ? 1.0f / d : 0.0f;
    } else {
        id = amax != 0.0f ? 127.0f / amax : 0.0f;
    }
    uint32_t wq[EPL / 4];
#pragma unroll
    for (int g = 0; g < EPL / 4; ++g) {
        uint32_t acc = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float v = f[4 * g + e] * id;
            float       q;
            if constexpr (ROUND == MI_Q8_0_REF) {
                q = round_half_away(v);
            } else {
                q = __builtin_amdgcn_fmed3f(__builtin_rintf(v), -128.0f, 127.0f);  // saturate like packs
            }
            acc |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        wq[g] = acc;
    }
    // EPL quants at byte 34*bi + 2 + EPL*sub (2-byte aligned)
    char *     bp = drow + (size_t) bi * 34;
    uint16_t * qp = (uint16_t *) (bp + 2 + sub * EPL);
#pragma unroll
    for (int g = 0; g < EPL / 4; ++g) {
        qp[2 * g]     = (uint16_t) (wq[g] & 0xffffu);
        qp[2 * g + 1] = (uint16_t) (wq[g] >> 16);
    }
    if (sub == 0) {
        *(uint16_t *) bp = f32_to_f16_bits(d);
    }
}

// Q8_0 destinations, staged: each wave owns a tile of 32 consecutive blocks
// (in work order). Its lanes first load the tile's source bytes as 16-byte
// chunks, lane-contiguous (every load instruction covers whole cache lines,
// whatever rows the tile spans), into LDS; then lane pairs quantize one block
// each (16 elements per lane) from LDS and store the quants and the scale.
template <int TI, int ROUND>
__global__ void __launch_bounds__(256) k_row_q8_lds(const RowCopy K, const RowCopy V, uint32_t nbk, uint32_t nbv,
                                                    uint32_t wg_k, uint32_t nbpr, FastDiv dnbpr) {
    constexpr int  EI  = TT<TI>::ES;
    constexpr int  VEC = TT<TI>::VEC;    // elements per 16-byte chunk
    constexpr int  CPB = 32 / VEC;       // chunks per block
    constexpr int  CPL = 32 * CPB / 64;  // chunks per lane per tile (F32: 4, BF16/F16: 2)
    __shared__ uint4 tile[4][32 * CPB];
    const int      lane = threadIdx.x & 63;
    const uint32_t wv   = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // workgroups [0, wg_k) store K, the rest V: the choice is uniform
    const bool      isv   = blockIdx.x >= wg_k;
    const RowCopy & R     = isv ? V : K;
    const uint32_t  total = isv ? nbv : nbk;
    const uint32_t  t0    = ((isv ? blockIdx.x - wg_k : blockIdx.x) * 4 + wv) * 32;  // first block of the tile
    if (t0 >= total) {
        return;  // whole wave
    }

    // 1. lane-contiguous chunk loads, all issued before any is used: blocks
    //    past the end re-load the last block (in bounds) and are never read
    uint4 v[CPL];
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        const int      c  = lane + 64 * k;
        const uint32_t gt = t0 + c / CPB;
        const uint32_t g  = gt < total ? gt : total - 1;
        const uint32_t w  = dnbpr.div(g);
        const uint32_t bi = g - w * nbpr;
        v[k]              = ld16(src_ptr(R, w) + (size_t) (bi * 32 + (c % CPB) * VEC) * EI);
    }
    // this lane pair's block and destination row (the slot lookup overlaps the loads)
    const int      j   = lane >> 1;
    const int      sub = lane & 1;
    const uint32_t g   = t0 + j;
    const uint32_t gc  = g < total ? g : total - 1;
    const uint32_t w   = dnbpr.div(gc);
    const uint32_t bi  = gc - w * nbpr;
    const char *   srow;
    char *         drow;
    bool           bad;
    row_ptrs(R, w, srow, drow, bad);
#pragma unroll
    for (int k = 0; k < CPL; ++k) {
        tile[wv][lane + 64 * k] = v[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();

    // 2. one block per lane pair
    if (g >= total) {
        return;  // whole pairs; nothing below synchronizes
    }
    if (bad) {
        if (sub == 0 && bi == 0 && R.d_err) {
            atomicAdd(R.d_err, 1);
        }
        return;
    }
    float f[16];
#pragma unroll
    for (int k = 0; k < 16 / VEC; ++k) {
        unpack16<TI>(tile[wv][j * CPB + sub * (CPB / 2) + k], f + VEC * k);
    }
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        amax = fmaxf(amax, fabsf(f[e]));
    }
    amax          = group_max<2>(amax);
    const float d = div127(amax);
    float       id;
    if constexpr (ROUND == MI_Q8_0_REF) {
        id = d != 0.0f ? 1.0f / d : 0.0f;
    } else {
        id = amax != 0.0f ? 127.0f / amax : 0.0f;
    }
    uint32_t wq[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
        uint32_t acc = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float x = f[4 * q4 + e] * id;
            float       q;
            if constexpr (ROUND == MI_Q8_0_REF) {
                q = round_half_away(x);
            } else {
                q = __builtin_amdgcn_fmed3f(__builtin_rintf(x), -128.0f, 127.0f);  // saturate like packs
            }
            acc |= ((uint32_t) (int32_t) q & 0xffu) << (8 * e);
        }
        wq[q4] = acc;
    }
    char *     bp = drow + (size_t) bi * 34;
    uint16_t * qp = (uint16_t *) (bp + 2 + sub * 16);  // 16 quants, 2-byte aligned
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
        qp[2 * q4]     = (uint16_t) (wq[q4] & 0xffffu);
        qp[2 * q4 + 1] = (uint16_t) (wq[q4] >> 16);
    }
    if (sub == 0) {
        *(uint16_t *) bp = f32_to_f16_bits(d);
    }
}

// F32 / F16 / BF16 destinations: 4 lanes per 32 elements, 8 per lane.
template <int TI, int TO>
__global__ void __launch_bounds__(256) k_row_copy(const RowCopy K, const RowCopy V, uint32_t nbk, uint32_t total,
                                                  uint32_t nbpr, FastDiv dnbpr) {
    constexpr int  EI  = TT<TI>::ES;
    const uint32_t gid = blockIdx.x * 256u + threadIdx.x;
    const uint32_t blk = gid >> 2;
    const int      sub = gid & 3;
    if (blk >= total) {
        return;
    }
    const bool      isv = blk >= nbk;
    const RowCopy & R   = isv ? V : K;
    const uint32_t  b2  = isv ? blk - nbk : blk;
    const uint32_t  w   = dnbpr.div(b2);
    const uint32_t  bi  = b2 - w * nbpr;
    const int       e0  = (int) bi * 32 + sub * 8;
    const char *    src;
    char *          drow;
    bool            bad;
    row_ptrs(R, w, src, drow, bad);
    float f[8];
    load8<TI>(src + (size_t) e0 * EI, f);
    if (bad) {
        if (sub == 0 && bi == 0 && R.d_err) {
            atomicAdd(R.d_err, 1);
        }
        return;
    }
    if constexpr (TO == MI_TYPE_F32) {
        // two 16-byte stores per lane, 16 bytes apart: plain (cached) stores so
        // the halves of each line merge in L2 before they reach HBM
        uint4 * p = (uint4 *) (drow + (size_t) e0 * 4);
        p[0]      = pack16<MI_TYPE_F32>(f);
        p[1]      = pack16<MI_TYPE_F32>(f + 4);
    } else {
        store_vec<TO, 8>(drow + (size_t) e0 * 2, f);
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
        const char *    srow;
        char *          drow;
        bool            bad;
        row_ptrs(R, row, srow, drow, bad);
        if (bad) {
            if (c == 0 && R.d_err) {
                atomicAdd(R.d_err, 1);
            }
            continue;
        }
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
        if constexpr (TO == MI_TYPE_Q8_0) {
#if MI_Q8_LDS
            const uint32_t nbv  = total - nbk;
            const uint32_t wg_k = (nbk + 127) / 128;  // 4 waves x 32 blocks per workgroup
            const uint32_t grid = wg_k + (nbv + 127) / 128;
            MI_LAUNCH((k_row_q8_lds<TI, ROUND>), dim3(grid), dim3(256), 0, s, K, Vr, nbk, nbv, wg_k, nbpr,
                               FastDiv(nbpr));
#else
            const uint32_t grid = (total * MI_Q8_LPB + 255) / 256;
            MI_LAUNCH((k_row_q8<TI, ROUND>), dim3(grid), dim3(256), 0, s, K, Vr, nbk, total, nbpr,
                               FastDiv(nbpr));
#endif
        } else {
            const uint32_t grid = (total * 4 + 255) / 256;
            MI_LAUNCH((k_row_copy<TI, TO>), dim3(grid), dim3(256), 0, s, K, Vr, nbk, total, nbpr,
                               FastDiv(nbpr));
        }
        return MI_OK;
    }
    const int      per_row = TO == MI_TYPE_Q8_0 ? K.ne0 / 32 : K.ne0;
    const uint64_t nk      = (uint64_t) K.rows * per_row;
    const uint64_t total   = nk + (V ? (uint64_t) V->rows * per_row : 0);
    uint64_t       grid    = (total + 255) / 256;
    const uint64_t cap     = (uint64_t) num_cus() * 32;
    grid                   = grid > cap ? cap : (grid ? grid : 1);
    MI_LAUNCH((k_row_copy_generic<TI, TO, ROUND>), dim3((uint32_t) grid), dim3(256), 0, s, K, Vr, nk, total,
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
    (void) tin;
    const int sa = 16;  // 8-element source loads: 16-byte vectors
    if (!aligned(R.src, sa) || R.sr.s1 % sa || R.sr.s2 % sa || R.sr.s3 % sa) {
        return false;
    }
    if (tout == MI_TYPE_Q8_0) {  // 16-bit stores into 34-byte blocks
        return aligned(R.dst, 2) && (R.kv ? (R.cnb1 % 2 == 0 && R.cnb2 % 2 == 0 && R.cnb3 % 2 == 0)
                                          : (R.dr.s1 % 2 == 0 && R.dr.s2 % 2 == 0 && R.dr.s3 % 2 == 0));
    }
    const int da = 16;  // 8-element destination stores
    return aligned(R.dst, da) && (R.kv ? (R.cnb1 % da == 0 && R.cnb2 % da == 0 && R.cnb3 % da == 0)
                                       : (R.dr.s1 % da == 0 && R.dr.s2 % da == 0 && R.dr.s3 % da == 0));
}

int launch_row_copy(const RowCopy & K, const RowCopy * V, int tin, int tout, int rounding, hipStream_t s) {
    if (K.rows == 0 || K.ne0 == 0) {
        return MI_OK;
    }
    bool fast = K.ne0 % 32 == 0 && row_aligned(K, tin, tout) && (!V || row_aligned(*V, tin, tout));
    fast      = fast && (uint64_t) (K.rows + (V ? V->rows : 0)) * (K.ne0 / 32) * 4 < (1ull << 31) &&
           (tout != MI_TYPE_Q8_0 || K.ne0 % 32 == 0);
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
